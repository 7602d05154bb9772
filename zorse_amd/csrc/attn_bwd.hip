// Flash-attention backward for gfx950 (bf16 / fp16 storage), atomic-free.
//
// Two kernels, both on the caller's stream, in this order:
//  1. attn_bwd_dq: Q-stationary (the forward's structure).  A workgroup owns
//     128 queries of one (batch, q-head), 32 per wave with Q and dO rows in
//     registers, and streams 64-key tiles of K and V through LDS:
//       S^T = K Q^T,  dP^T = V dO^T,  dS^T = P^T (dP^T - delta),
//       dQ^T += K^T dS^T              (K^T read transposed from LDS)
//     Each lane owns one query, so lse and delta are per-lane scalars; the
//     kernel first forms delta = rowsum(dO o O) from the dO row it holds and
//     one read of O, and stores it with the log2-domain LSE for kernel 2.
//  2. attn_bwd_dkdv: KV-stationary.  A workgroup owns 128 keys of one
//     (batch, kv-head) -- 32 keys per wave, that wave's K rows held in
//     registers and its V rows in LDS as MFMA B operands -- and loops over
//     32-query blocks of every q-head in the GQA group (the group reduction of
//     dK / dV happens in the accumulators; repeat_kv is never materialised).
//     Within 256 registers, two workgroups share a CU.  Per block:
//       S  = Q K^T,  dP = dO V^T      (A = Q / dO rows from LDS)
//       P  = exp2(S scale log2e - lse log2e),  dS = P (dP - delta)
//       dV^T += dO^T P,  dK^T += Q^T dS
//     with dO^T / Q^T read transposed straight from the row-major LDS tiles
//     (ds_read_tr16_b64) and P / dS fed from the score accumulators as the B
//     operand (a fixed query permutation, matched by the transposed reads).
// dQ is produced by its own pass instead of fp32 atomics into a shared
// accumulator: S and dP are recomputed there (4 of the 14 d-length products
// per pair), which costs less than device-scope atomic traffic (measured:
// fp32 atomic adds into an L2-sized accumulator run at ~0.3 TB/s here) and
// keeps the result deterministic.  With RoPE (zk_attn_bwd_rope) both
// epilogues apply the rotation's transpose before storing dQ / dK.
#include <type_traits>

#include "attn_common.h"
#include "vec.h"

namespace zk {

int check_attn_desc(const zk_attn_desc* d, const char* who, bool bwd);
void fill_args(AttnArgs& a, const zk_attn_desc* d);

// ----------------------------------------------------------------- prep ----
// fp32 path: 8 lanes per (b, q, h) row; each lane covers d/8 elements.
// Writes delta = rowsum(dO o O) and lse2 = lse * log2(e) (+inf for an empty
// row, so that exp2(s - lse2) = 0), both fp32 [B, Hq, Sq].  (The MFMA path
// forms both inside attn_bwd_dq.)
template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_prep(AttnArgs a) {
  const int64_t rows = a.B * a.Sq * a.Hq;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t row = gid >> 3;
  const int sub = threadIdx.x & 7;
  float acc = 0.f;
  int64_t b = 0, q = 0, h = 0;
  if (row < rows) {
    h = row % a.Hq;
    const int64_t bq = row / a.Hq;
    q = bq % a.Sq;
    b = bq / a.Sq;
    const T* Or = static_cast<const T*>(a.o) + b * a.o_sb + q * a.o_ss + h * a.o_sh;
    const T* Dr = static_cast<const T*>(a.dout) + b * a.o_sb + q * a.o_ss + h * a.o_sh;
    for (int64_t e = sub; e < a.d; e += 8) acc = fmaf(to_f32(Or[e]), to_f32(Dr[e]), acc);
  }
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  acc += __shfl_xor(acc, 4, 64);
  if (row < rows && sub == 0) {
    const int64_t i = (b * a.Hq + h) * a.Sq + q;
    a.delta[i] = acc;
    const float l = a.lse[i];
    a.lse2[i] = l == -INFINITY ? INFINITY : l * kLog2e;
  }
}

// ------------------------------------------------------------- dK / dV -----
template <int D>
struct DkdvCfg {
  // 4 waves, two workgroups per CU (8 waves and 256 keys per workgroup, one
  // workgroup per CU, measured 2-5 % slower)
  static constexpr int BK = 128;              // keys per workgroup (32 per wave)
  static constexpr int MQ = 32;               // queries per block
  static constexpr int MB = MQ / 32;          // 32-row MFMA blocks per query block
};

// kFull: Sq is a multiple of the query block, so no block runs past the end.
template <typename T, int D, bool kFull>
__global__ __launch_bounds__(256, 2) void attn_bwd_dkdv(AttnArgs a) {
  typedef DkdvCfg<D> C;
  typedef Mfma<T> M;
  typedef typename M::vec8 V8;
  constexpr int BK = C::BK, MQ = C::MQ;
  // Q / dO tiles double-buffered (swizzled rows); each wave keeps its own copy
  // of the block's lse2 / delta vectors so every wave issues the same loads.
  // Q / dO tiles of the two stages, each its own array: the compiler then sees
  // that the next stage's asynchronous loads do not alias this stage's reads
  // (and adds no wait for them)
  __shared__ __attribute__((aligned(16))) T Q0[MQ * D], Q1[MQ * D], dO0[MQ * D], dO1[MQ * D];
  __shared__ __attribute__((aligned(16))) float lse2s[2][4][64];  // 64 lanes load, MQ used
  // V rows of each wave's 32 keys (the B operand of dP), swizzled like the tiles
  __shared__ __attribute__((aligned(16))) T Vw[4][32 * D];
  __shared__ __attribute__((aligned(16))) float dels[2][4][64];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int64_t nbh = a.B * a.Hkv;
  const int64_t bid = blockIdx.x;
  const int64_t kt = bid / nbh;  // low key tiles carry the most causal work: first
  const int64_t bh = bid % nbh;
  const int64_t b = bh / a.Hkv, hk = bh % a.Hkv;
  const int64_t n_rep = a.Hq / a.Hkv;
  const int64_t k0 = kt * BK;
  const int64_t kw0 = k0 + 32 * wave;
  const int64_t my_key = kw0 + l32;
  const float c2 = a.scale_log2;
  // Queries that see this lane's key form one range [vis_lo, vis_lo + vis_span]
  // (causal: from the key on; window: the W queries starting at the key;
  // below Sq), so the element mask is one unsigned compare per score.
  int vis_lo, vis_span;
  {
    const int ik = static_cast<int>(my_key);
    int hi = static_cast<int>(a.Sq) - 1;
    if (a.window > 0 && ik + static_cast<int>(a.window) - 1 < hi) hi = ik + static_cast<int>(a.window) - 1;
    vis_lo = a.causal ? ik : 0;
    vis_span = hi - vis_lo;
    if (vis_span < 0 || my_key >= a.Skv) {
      vis_lo = 0x40000000;
      vis_span = 0;
    }
  }

  const T* Kp = static_cast<const T*>(a.k) + b * a.k_sb + hk * a.k_sh;
  const T* Vp = static_cast<const T*>(a.v) + b * a.v_sb + hk * a.v_sh;

  // B operands of S = Q K^T and dP = dO V^T: lane holds row my_key.  K stays
  // in registers; V goes to this wave's LDS rows (read back per step), which
  // keeps the kernel within 256 registers (two waves per SIMD).
  V8 kreg[D / 16];
  T* Vme = Vw[wave];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    V8 vv;
    if (my_key < a.Skv) {
      kreg[ks] = *reinterpret_cast<const V8*>(Kp + my_key * a.k_ss + 16 * ks + 8 * g);
      vv = *reinterpret_cast<const V8*>(Vp + my_key * a.v_ss + 16 * ks + 8 * g);
    } else {
      kreg[ks] = V8{};
      vv = V8{};
    }
    *reinterpret_cast<V8*>(&Vme[tile_off<D>(l32, 16 * ks + 8 * g)]) = vv;
  }

  f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
  for (int nt = 0; nt < D / 32; ++nt) {
    dk[nt] = f32x16{};
    dv[nt] = f32x16{};
  }
  // LDS byte offsets, derived on the fly from two per-lane bases (the swizzle
  // XORs chunk indices, and a row's chunk bits never overlap its row bits, so
  // moving to another chunk is an XOR by a constant):
  //  * row reads of this lane's row l32, chunk 2 ks + g: rbase ^ (ks << 5);
  //  * transposed reads (ds_read_tr16_b64) of 32-column block nt for the
  //    16-query step kk = 0: keys 4 g .. at tbase ^ (nt << 6), keys 8 + 4 g ..
  //    at that ^ 32 (their swizzle differs by 2 chunks) plus 8 rows.
  // Two registers instead of one per operand slot keep the kernel within 256.
  static_assert(MQ == 32, "one 32-row block per step");
  const int rbase = 2 * tile_off<D>(l32, 8 * g);
  const int tbase = 2 * tile_off<D>(4 * g + ((lane & 15) >> 2), 16 * ((lane >> 4) & 1) + 4 * (lane & 3));

  // queries that can see keys [k0, k0 + BK)
  int64_t q_lo = 0, q_hi = a.Sq;
  if (a.causal) q_lo = k0;
  if (a.window > 0 && k0 + BK - 1 + a.window < q_hi) q_hi = k0 + BK - 1 + a.window;
  const int64_t qb_lo = q_lo / MQ;
  const int64_t qb_hi = q_hi > q_lo ? (q_hi + MQ - 1) / MQ : qb_lo;
  const int64_t nqb = qb_hi - qb_lo;
  const int64_t n_iter = nqb * n_rep;

  TileLoader<T, D, MQ> qload, dload;
  qload.init(a.q_ss);
  dload.init(a.o_ss);
  // iteration it covers query block qb_lo + it % nqb of q-head hk * n_rep +
  // it / nqb; (qbi, hr) below track that pair without dividing
  auto issue = [&](int64_t qbi, int64_t hr, int st) {
    const int64_t hq = hk * n_rep + hr;
    const int64_t qb0 = qbi * MQ;
    const T* Qp = static_cast<const T*>(a.q) + b * a.q_sb + hq * a.q_sh;
    const T* Dp = static_cast<const T*>(a.dout) + b * a.o_sb + hq * a.o_sh;
    qload.issue(st ? Q1 : Q0, Qp, a.q_ss, qb0, a.Sq, kFull);
    dload.issue(st ? dO1 : dO0, Dp, a.o_ss, qb0, a.Sq, kFull);
    int64_t qi = qb0 + lane;
    if (qi > a.Sq - 1) qi = a.Sq - 1;
    const int64_t r0 = (b * a.Hq + hq) * a.Sq + qb0;
    const uint32_t off = static_cast<uint32_t>((qi - qb0) * 4);
    dma_lds<4>(raw_rsrc(a.lse2 + r0), off, 0, &lse2s[st][wave][0]);
    dma_lds<4>(raw_rsrc(a.delta + r0), off, 0, &dels[st][wave][0]);
  };

  // transposed MFMA operand of tile X for 16-query step kk (see lds_tr_operand)
  auto tr_at = [&](const T* X, int off, int kk) __attribute__((always_inline)) {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    const char* base = reinterpret_cast<const char*>(X) + kk * 16 * D * 2;
    const s16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + off));
    const s16x4 x1 =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + 8 * D * 2 + (off ^ 32)));
    const s16x8 w = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
    return __builtin_bit_cast(V8, w);
  };

  // One pipeline step on LDS stage ST (compile-time: immediate LDS offsets).
  auto step = [&](auto stage_tag, int64_t qbi, int64_t nxt_qbi, int64_t nxt_hr, bool has_next) {
    constexpr int st = decltype(stage_tag)::value;
    const int64_t qb0 = qbi * MQ;
    wait_vmcnt<0>();  // this wave's loads of this block have landed
    __syncthreads();  // ... and every wave's; all are done with the other stage
    if (has_next) issue(nxt_qbi, nxt_hr, st ^ 1);

    // wave-uniform classification of this (query block, 32 keys) tile
    bool skip = false, need_mask = kw0 + 31 >= a.Skv || qb0 + MQ > a.Sq;
    if (a.causal) {
      if (kw0 > qb0 + MQ - 1) skip = true;
      if (kw0 + 31 > qb0) need_mask = true;
    }
    if (a.window > 0) {
      if (kw0 + 31 <= qb0 - a.window) skip = true;
      if (kw0 <= qb0 + MQ - 1 - a.window) need_mask = true;
    }
    if (skip) return;
    const T* Qt = st ? Q1 : Q0;
    const T* dOt = st ? dO1 : dO0;
    // opaque per-step copies of the bases: the addresses derived from them are
    // recomputed in the step instead of being kept live across the loop
    int rb = rbase, tb = tbase;
    asm volatile("" : "+v"(rb), "+v"(tb));
    const float* l2v = lse2s[st][wave];
    const float* dlv = dels[st][wave];
    const int qb32 = static_cast<int>(qb0);

    // S and dP of the 32-query half mb (rows 32 mb .. +31 of the block)
    auto scores = [&](int mb, f32x16& sv, f32x16& dpv) {
      sv = f32x16{};
      dpv = f32x16{};
      // each step's Q operand read one step ahead, before the MFMAs of the
      // step it follows (the fences keep the compiler from sinking it)
      V8 qa = *reinterpret_cast<const V8*>(reinterpret_cast<const char*>(Qt) + rb);
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
        const int ro = rb ^ (ks << 5);
        const V8 da = *reinterpret_cast<const V8*>(reinterpret_cast<const char*>(dOt) + ro);
        const V8 vb = *reinterpret_cast<const V8*>(reinterpret_cast<const char*>(Vme) + ro);
        V8 qn = qa;
        if (ks + 1 < D / 16)
          qn = *reinterpret_cast<const V8*>(reinterpret_cast<const char*>(Qt) + (rb ^ ((ks + 1) << 5)));
        __builtin_amdgcn_sched_barrier(0);
        sv = M::mma(qa, kreg[ks], sv);
        dpv = M::mma(da, vb, dpv);
        qa = qn;
      }
    };
    // P and dS of half mb, packed as the B operands of two 16-query MFMA steps;
    // element j is query 32 mb + 8 (j/4) + 4 g + j%4
    auto probs = [&](auto mask_tag, int mb, const f32x16& sv, const f32x16& dpv, V8 (&pb)[2],
                     V8 (&sb)[2]) {
      constexpr bool kMask = decltype(mask_tag)::value;
#pragma unroll
      for (int a4 = 0; a4 < 4; ++a4) {
        const int r0 = 32 * mb + 8 * a4 + 4 * g;
        const float4 l4 = *reinterpret_cast<const float4*>(&l2v[r0]);
        const float4 d4 = *reinterpret_cast<const float4*>(&dlv[r0]);
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
        const float dl[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = 4 * a4 + e;
          float p = __builtin_amdgcn_exp2f(fmaf(sv[j], c2, -lv[e]));
          if (kMask && static_cast<unsigned>(qb32 + r0 + e - vis_lo) > static_cast<unsigned>(vis_span))
            p = 0.f;
          pb[j >> 3][j & 7] = static_cast<T>(p);
          sb[j >> 3][j & 7] = static_cast<T>(p * (dpv[j] - dl[e]));
        }
      }
    };
    // dV^T += dO^T P ; dK^T += Q^T dS over the two 16-query steps of half mb.
    // Step kk covers queries 16 kk + perm: lane half g holds queries
    // 16 kk + 4 g + 0..3 and 16 kk + 8 + 4 g + 0..3.
    auto accumulate = [&](int mb, const V8 (&pb)[2], const V8 (&sb)[2]) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kk = 2 * mb + h;
#pragma unroll
        for (int nt = 0; nt < D / 32; ++nt) {
          const V8 dA = tr_at(dOt, tb ^ (nt << 6), kk);
          dv[nt] = M::mma(dA, pb[h], dv[nt]);
          const V8 qA = tr_at(Qt, tb ^ (nt << 6), kk);
          dk[nt] = M::mma(qA, sb[h], dk[nt]);
        }
      }
    };
    // One 32-query block per step; the other wave on the SIMD (two
    // workgroups per CU) covers this wave's VALU and LDS latencies.
    auto body = [&](auto mask_tag) {
      f32x16 s0, dp0;
      V8 pb0[2], sb0[2];
      scores(0, s0, dp0);
      probs(mask_tag, 0, s0, dp0, pb0, sb0);
      accumulate(0, pb0, sb0);
    };
    if (need_mask)
      body(std::true_type{});
    else
      body(std::false_type{});
  };

  int64_t qbi = qb_lo, hr = 0;
  auto advance = [&](int64_t& q, int64_t& h) {
    if (++q == qb_hi) {
      q = qb_lo;
      ++h;
    }
  };
  if (n_iter > 0) issue(qbi, hr, 0);
  for (int64_t it = 0; it < n_iter; it += 2) {
    int64_t nq = qbi, nh = hr;
    advance(nq, nh);
    step(std::integral_constant<int, 0>{}, qbi, nq, nh, it + 1 < n_iter);
    qbi = nq;
    hr = nh;
    if (it + 1 < n_iter) {
      advance(nq, nh);
      step(std::integral_constant<int, 1>{}, qbi, nq, nh, it + 2 < n_iter);
      qbi = nq;
      hr = nh;
    }
  }

  // dK = scale (Q^T dS)^T, dV = (dO^T P)^T: lane holds key my_key and
  // d rows 32 nt + 8 a4 + 4 g + 0..3 (4 consecutive elements).
  if (my_key < a.Skv) {
    if (a.rope_cos != nullptr) rope_inverse_regs<D>(dk, a, my_key, g);
    typedef T T4 __attribute__((ext_vector_type(4)));
    T* dkp = static_cast<T*>(a.dk) + b * a.dk_sb + hk * a.dk_sh + my_key * a.dk_ss;
    T* dvp = static_cast<T*>(a.dv) + b * a.dv_sb + hk * a.dv_sh + my_key * a.dv_ss;
#pragma unroll
    for (int nt = 0; nt < D / 32; ++nt)
#pragma unroll
      for (int a4 = 0; a4 < 4; ++a4) {
        const int d0 = 32 * nt + 8 * a4 + 4 * g;
        T4 wk, wv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          wk[e] = static_cast<T>(dk[nt][4 * a4 + e] * a.scale);
          wv[e] = static_cast<T>(dv[nt][4 * a4 + e]);
        }
        *reinterpret_cast<T4*>(dkp + d0) = wk;
        *reinterpret_cast<T4*>(dvp + d0) = wv;
      }
  }
  if (a.dk_t != nullptr) {
    // dK^T / dV^T rows hk D .. +D-1, token columns b Skv + k0 ..; the V rows'
    // LDS (128 x D elements) holds the tile once every wave is past its last step
    __syncthreads();
    const int64_t left = a.Skv - k0;
    const int nc = static_cast<int>(left < BK ? left : BK);
    const int64_t off = hk * D * a.t_ld + b * a.Skv + k0;
    T* tile = &Vw[0][0];  // all D rows in one array (the other pointers are unused)
    store_rows_transposed<T, D, BK, D>(dk, a.scale, tile, tile, tile, tile,
                                       static_cast<T*>(a.dk_t) + off, a.t_ld, nc);
    store_rows_transposed<T, D, BK, D>(dv, 1.f, tile, tile, tile, tile,
                                       static_cast<T*>(a.dv_t) + off, a.t_ld, nc);
  }
}

// ------------------------------------------------------------------ dQ -----
template <int D>
struct DqCfg {
  // 4 waves, two workgroups per CU (8 waves sharing each K / V tile, as the
  // forward does, measured equal here: this kernel is not bound by its tile loads)
  static constexpr int NW = 4;
  static constexpr int NT = 64 * NW;
  static constexpr int BM = 32 * NW;          // queries per workgroup (32 per wave)
  static constexpr int BN = 64;               // keys per tile
  static constexpr int PF = 2;                // LDS operand reads in flight
};

// kFull: Skv is a multiple of the key tile, so no tile runs past the end.
template <typename T, int D, bool kFull>
__global__ __launch_bounds__(256, 2) void attn_bwd_dq(AttnArgs a, int64_t n_qt) {
  typedef DqCfg<D> C;
  typedef Mfma<T> M;
  typedef typename M::vec8 V8;
  constexpr int BM = C::BM, BN = C::BN, NT = C::NT;
  // swizzled rows; each stage its own array, so the compiler sees that the
  // next tile's asynchronous loads do not alias this tile's reads
  __shared__ __attribute__((aligned(16))) T K0[BN * D], K1[BN * D], V0[BN * D], V1[BN * D];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int64_t nbh = a.B * a.Hq;
  const int64_t bid = blockIdx.x;
  const int64_t qt = n_qt - 1 - bid / nbh;  // heaviest (last) query tiles first
  const int64_t bh = bid % nbh;
  const int64_t b = bh / a.Hq, hq = bh % a.Hq;
  const int64_t hk = hq / (a.Hq / a.Hkv);
  const int64_t q0 = qt * BM;
  const int64_t qw0 = q0 + 32 * wave;
  const int64_t my_q = qw0 + l32;
  const float c2 = a.scale_log2;
  // keys visible to this lane's query: [vis_lo, vis_lo + vis_span]
  int vis_lo, vis_span;
  {
    const int iq = static_cast<int>(my_q);
    int hi = static_cast<int>(a.Skv) - 1;
    if (a.causal && iq < hi) hi = iq;
    const int lo = a.window > 0 ? iq - static_cast<int>(a.window) + 1 : 0;
    vis_lo = lo > 0 ? lo : 0;
    vis_span = hi - vis_lo;
    if (vis_span < 0 || my_q >= a.Sq) {
      vis_lo = 0x40000000;
      vis_span = 0;
    }
  }

  const T* Qp = static_cast<const T*>(a.q) + b * a.q_sb + hq * a.q_sh;
  const T* Dp = static_cast<const T*>(a.dout) + b * a.o_sb + hq * a.o_sh;
  const T* Kp = static_cast<const T*>(a.k) + b * a.k_sb + hk * a.k_sh;
  const T* Vp = static_cast<const T*>(a.v) + b * a.v_sb + hk * a.v_sh;

  // B operands of S^T = K Q^T and dP^T = V dO^T: lane holds query my_q.
  V8 qreg[D / 16], dreg[D / 16];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    if (my_q < a.Sq) {
      qreg[ks] = *reinterpret_cast<const V8*>(Qp + my_q * a.q_ss + 16 * ks + 8 * g);
      dreg[ks] = *reinterpret_cast<const V8*>(Dp + my_q * a.o_ss + 16 * ks + 8 * g);
    } else {
      qreg[ks] = V8{};
      dreg[ks] = V8{};
    }
  }
  // delta = rowsum(dO o O) and the log2-domain LSE of this lane's query,
  // computed here (each lane holds half of the row: d = 16 ks + 8 g + 0..7)
  // and stored for the dK / dV kernel, which runs after this one
  float lse2 = INFINITY, del = 0.f;
  {
    const T* Op = static_cast<const T*>(a.o) + b * a.o_sb + hq * a.o_sh;
    float part = 0.f;
    if (my_q < a.Sq) {
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
        const V8 ov = *reinterpret_cast<const V8*>(Op + my_q * a.o_ss + 16 * ks + 8 * g);
#pragma unroll
        for (int e = 0; e < 8; ++e) part = fmaf(to_f32(ov[e]), to_f32(dreg[ks][e]), part);
      }
    }
    del = part + other_half(part);
    if (my_q < a.Sq) {
      const int64_t i = (b * a.Hq + hq) * a.Sq + my_q;
      const float l = a.lse[i];
      lse2 = l == -INFINITY ? INFINITY : l * kLog2e;
      if (g == 0) {
        a.delta[i] = del;
        a.lse2[i] = lse2;
      }
    }
  }

  int64_t kv_lo = 0, kv_hi = a.Skv;
  if (a.causal && kv_hi > q0 + BM) kv_hi = q0 + BM;
  if (a.window > 0 && q0 - a.window + 1 > kv_lo) kv_lo = q0 - a.window + 1;
  const int64_t t_lo = kv_lo / BN;
  const int64_t t_hi = kv_hi > kv_lo ? (kv_hi + BN - 1) / BN : t_lo;

  TileLoader<T, D, BN, NT> kload, vload;
  kload.init(a.k_ss);
  vload.init(a.v_ss);
  auto issue = [&](int64_t kb0, int st) {
    kload.issue(st ? K1 : K0, Kp, a.k_ss, kb0, a.Skv, kFull);
    vload.issue(st ? V1 : V0, Vp, a.v_ss, kb0, a.Skv, kFull);
  };
  // LDS byte offsets from two per-lane bases, as in the dK/dV kernel: row
  // l32 + 32 tt, chunk 2 ks + g at (rbase ^ (ks << 5)) + tt rows; transposed
  // K reads of block nt at (tbase ^ (nt << 6)) + kk rows (keys 4 g ..) and at
  // that ^ 32 plus 8 rows (keys 8 + 4 g ..)
  const int rbase = 2 * tile_off<D>(l32, 8 * g);
  const int tbase = 2 * tile_off<D>(4 * g + ((lane & 15) >> 2), 16 * ((lane >> 4) & 1) + 4 * (lane & 3));

  f32x16 dq[D / 32];
#pragma unroll
  for (int nt = 0; nt < D / 32; ++nt) dq[nt] = f32x16{};

  // One pipeline step on LDS stage ST (compile-time: immediate LDS offsets).
  auto step = [&](auto stage_tag, int64_t t) {
    constexpr int st = decltype(stage_tag)::value;
    const int64_t kb0 = t * BN;
    wait_vmcnt<0>();  // this wave's loads of tile t have landed
    __syncthreads();  // ... and every wave's; all are done with the other stage
    if (t + 1 < t_hi) issue(kb0 + BN, st ^ 1);

    bool skip = false, need_mask = kb0 + BN > a.Skv || qw0 + 31 >= a.Sq;
    if (a.causal) {
      if (kb0 > qw0 + 31) skip = true;
      if (kb0 + BN - 1 > qw0) need_mask = true;
    }
    if (a.window > 0) {
      if (kb0 + BN - 1 <= qw0 - a.window) skip = true;
      if (kb0 <= qw0 + 31 - a.window) need_mask = true;
    }
    if (skip) return;
    const T* Kt = st ? K1 : K0;
    const T* Vt = st ? V1 : V0;
    int rb = rbase, tb = tbase;  // opaque per-step copies (addresses derived in the step)
    asm volatile("" : "+v"(rb), "+v"(tb));

    // one 32-key block at a time: S^T and dP^T of keys kb0 + 32 tt .. +31,
    // its dS^T, then its two 16-key steps of dQ^T += K^T dS^T
#pragma unroll
    for (int tt = 0; tt < BN / 32; ++tt) {
      f32x16 s = f32x16{}, dp = f32x16{};
      // LDS operands are read PF MFMA steps ahead, each step fenced so that
      // the reads stay where they are placed (left alone, the compiler reads
      // each operand just before its MFMA and waits out the LDS latency)
      constexpr int PF = C::PF;
      auto rowread = [&](const T* X, int ks) __attribute__((always_inline)) {
        const int ro = (rb ^ (ks << 5)) + tt * 32 * D * 2;
        return *reinterpret_cast<const V8*>(reinterpret_cast<const char*>(X) + ro);
      };
      V8 kq[PF], vq[PF];
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        kq[i] = rowread(Kt, i);
        vq[i] = rowread(Vt, i);
      }
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
        __builtin_amdgcn_sched_barrier(0);
        const V8 kA = kq[ks % PF], vA = vq[ks % PF];
        if (ks + PF < D / 16) {
          kq[ks % PF] = rowread(Kt, ks + PF);
          vq[ks % PF] = rowread(Vt, ks + PF);
        }
        s = M::mma(kA, qreg[ks], s);
        dp = M::mma(vA, dreg[ks], dp);
      }
      __builtin_amdgcn_sched_barrier(0);
      // dS^T packed per 16-key MFMA step (key = kb0 + 32 tt + 8 (j/4) + 4 g + j%4)
      V8 sb[2];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float p = __builtin_amdgcn_exp2f(fmaf(s[j], c2, -lse2));
        if (need_mask) {
          const int rel = static_cast<int>(kb0) - vis_lo + 32 * tt + 8 * (j >> 2) + 4 * g + (j & 3);
          if (static_cast<unsigned>(rel) > static_cast<unsigned>(vis_span)) p = 0.f;
        }
        sb[j >> 3][j & 7] = static_cast<T>(p * (dp[j] - del));
      }
      // dQ^T += K^T dS^T  (K^T read transposed from the row-major K tile),
      // operands read PF MFMAs ahead
      auto trread = [&](int m) __attribute__((always_inline)) {
        typedef short s16x4 __attribute__((ext_vector_type(4)));
        typedef short s16x8 __attribute__((ext_vector_type(8)));
        typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
        const int kk = 2 * tt + m / (D / 32), nt = m % (D / 32);
        const char* kb = reinterpret_cast<const char*>(Kt) + kk * 16 * D * 2;
        const int off = tb ^ (nt << 6);
        const s16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(kb + off));
        const s16x4 x1 =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(kb + 8 * D * 2 + (off ^ 32)));
        const s16x8 w = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
        return __builtin_bit_cast(V8, w);
      };
      constexpr int NM = 2 * (D / 32);
      V8 tq[PF];
#pragma unroll
      for (int i = 0; i < PF; ++i) tq[i] = trread(i);
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        __builtin_amdgcn_sched_barrier(0);
        const V8 w = tq[m % PF];
        if (m + PF < NM) tq[m % PF] = trread(m + PF);
        dq[m % (D / 32)] = M::mma(w, sb[m / (D / 32)], dq[m % (D / 32)]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  if (t_lo < t_hi) issue(t_lo * BN, 0);
  for (int64_t t = t_lo; t < t_hi; t += 2) {
    step(std::integral_constant<int, 0>{}, t);
    if (t + 1 < t_hi) step(std::integral_constant<int, 1>{}, t + 1);
  }

  if (my_q < a.Sq) {
    if (a.rope_cos != nullptr) rope_inverse_regs<D>(dq, a, my_q, g);
    typedef T T4 __attribute__((ext_vector_type(4)));
    T* dqp = static_cast<T*>(a.dq) + b * a.dq_sb + hq * a.dq_sh + my_q * a.dq_ss;
#pragma unroll
    for (int nt = 0; nt < D / 32; ++nt)
#pragma unroll
      for (int a4 = 0; a4 < 4; ++a4) {
        const int d0 = 32 * nt + 8 * a4 + 4 * g;
        T4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = static_cast<T>(dq[nt][4 * a4 + e] * a.scale);
        *reinterpret_cast<T4*>(dqp + d0) = w;
      }
  }
  if (a.dq_t != nullptr) {
    // dQ^T rows hq D .. +D-1, token columns b Sq + q0 ..; the K / V stages
    // hold the tile once every wave is past its last step
    __syncthreads();
    const int64_t left = a.Sq - q0;
    store_rows_transposed<T, D, BM, BN * D / BM>(
        dq, a.scale, K0, K1, V0, V1, static_cast<T*>(a.dq_t) + hq * D * a.t_ld + b * a.Sq + q0,
        a.t_ld, static_cast<int>(left < BM ? left : BM));
  }
}

// ------------------------------------------------------------- fp32 path ---
// Simple per-row kernels for fp32 layers (small shapes, no MFMA).

// The inverse RoPE rotation of one row x[0 .. d) at sequence position `row`
// (the same pairings and formula as rope_inverse_regs).
__device__ __forceinline__ void rope_inverse_row(float* x, const AttnArgs& a, int64_t row) {
  int64_t pos = a.rope_pos != nullptr ? a.rope_pos[row] : row;
  if (pos < 0) pos = 0;
  if (pos > a.rope_npos - 1) pos = a.rope_npos - 1;
  const int64_t half = a.d / 2;
  const float* ct = a.rope_cos + pos * half;
  const float* st = a.rope_sin + pos * half;
  for (int64_t i = 0; i < half; ++i) {
    const int64_t ia = a.rope_interleaved ? 2 * i : i;
    const int64_t ib = a.rope_interleaved ? 2 * i + 1 : i + half;
    const float u = x[ia], w = x[ib];
    x[ia] = fmaf(u, ct[i], w * st[i]);
    x[ib] = fmaf(w, ct[i], -u * st[i]);
  }
}
template <int D>
__global__ __launch_bounds__(64) void attn_bwd_dq_f32(AttnArgs a) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
  if (row >= a.B * a.Hq * a.Sq) return;
  const int64_t qi = row % a.Sq, bh = row / a.Sq;
  const int64_t b = bh / a.Hq, hq = bh % a.Hq, hk = hq / (a.Hq / a.Hkv);
  const float* Q = static_cast<const float*>(a.q) + b * a.q_sb + hq * a.q_sh + qi * a.q_ss;
  const float* dO = static_cast<const float*>(a.dout) + b * a.o_sb + hq * a.o_sh + qi * a.o_ss;
  const float* K = static_cast<const float*>(a.k) + b * a.k_sb + hk * a.k_sh;
  const float* V = static_cast<const float*>(a.v) + b * a.v_sb + hk * a.v_sh;
  const float lse = a.lse[(b * a.Hq + hq) * a.Sq + qi];
  const float del = a.delta[(b * a.Hq + hq) * a.Sq + qi];
  float acc[D];
  for (int e = 0; e < a.d; ++e) acc[e] = 0.f;
  for (int64_t j = 0; j < a.Skv; ++j) {
    if (!attn_visible(qi, j, a.Skv, a.causal, a.window)) continue;
    const float* kr = K + j * a.k_ss;
    const float* vr = V + j * a.v_ss;
    float s = 0.f, dp = 0.f;
    for (int e = 0; e < a.d; ++e) {
      s = fmaf(Q[e], kr[e], s);
      dp = fmaf(dO[e], vr[e], dp);
    }
    const float p = expf(s * a.scale - lse);
    const float ds = p * (dp - del) * a.scale;
    for (int e = 0; e < a.d; ++e) acc[e] = fmaf(ds, kr[e], acc[e]);
  }
  if (a.rope_cos != nullptr) rope_inverse_row(acc, a, qi);
  float* dq = static_cast<float*>(a.dq) + b * a.dq_sb + hq * a.dq_sh + qi * a.dq_ss;
  for (int e = 0; e < a.d; ++e) dq[e] = acc[e];
}

template <int D>
__global__ __launch_bounds__(64) void attn_bwd_dkv_f32(AttnArgs a) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
  if (row >= a.B * a.Hkv * a.Skv) return;
  const int64_t kj = row % a.Skv, bh = row / a.Skv;
  const int64_t b = bh / a.Hkv, hk = bh % a.Hkv;
  const int64_t n_rep = a.Hq / a.Hkv;
  const float* K = static_cast<const float*>(a.k) + b * a.k_sb + hk * a.k_sh + kj * a.k_ss;
  const float* V = static_cast<const float*>(a.v) + b * a.v_sb + hk * a.v_sh + kj * a.v_ss;
  float dk[D], dv[D];
  for (int e = 0; e < a.d; ++e) { dk[e] = 0.f; dv[e] = 0.f; }
  for (int64_t r = 0; r < n_rep; ++r) {
    const int64_t hq = hk * n_rep + r;
    const float* Q = static_cast<const float*>(a.q) + b * a.q_sb + hq * a.q_sh;
    const float* dO = static_cast<const float*>(a.dout) + b * a.o_sb + hq * a.o_sh;
    for (int64_t qi = 0; qi < a.Sq; ++qi) {
      if (!attn_visible(qi, kj, a.Skv, a.causal, a.window)) continue;
      const float* qr = Q + qi * a.q_ss;
      const float* dr = dO + qi * a.o_ss;
      float s = 0.f, dp = 0.f;
      for (int e = 0; e < a.d; ++e) {
        s = fmaf(qr[e], K[e], s);
        dp = fmaf(dr[e], V[e], dp);
      }
      const float lse = a.lse[(b * a.Hq + hq) * a.Sq + qi];
      const float del = a.delta[(b * a.Hq + hq) * a.Sq + qi];
      const float p = expf(s * a.scale - lse);
      const float ds = p * (dp - del) * a.scale;
      for (int e = 0; e < a.d; ++e) {
        dv[e] = fmaf(p, dr[e], dv[e]);
        dk[e] = fmaf(ds, qr[e], dk[e]);
      }
    }
  }
  if (a.rope_cos != nullptr) rope_inverse_row(dk, a, kj);
  float* dkp = static_cast<float*>(a.dk) + b * a.dk_sb + hk * a.dk_sh + kj * a.dk_ss;
  float* dvp = static_cast<float*>(a.dv) + b * a.dv_sb + hk * a.dv_sh + kj * a.dv_ss;
  for (int e = 0; e < a.d; ++e) { dkp[e] = dk[e]; dvp[e] = dv[e]; }
}

}  // namespace zk

using namespace zk;

extern "C" int64_t zk_attn_bwd_workspace(const zk_attn_desc* desc) {
  if (desc == nullptr) return 0;
  const int64_t rows = desc->B * desc->Hq * desc->Sq;  // fp32 delta and lse2
  return 2 * rows * 4 + 512;
}

namespace zk {
struct RopeInv {
  const float* cos;
  const float* sin;
  int64_t n_pos;
  const int64_t* positions;
  int pairing;
};

struct TransposedOut {
  void* dq_t;
  void* dk_t;
  void* dv_t;
  int64_t ld;
};

static int attn_bwd_impl(const char* who, const zk_attn_desc* desc, const void* q,
                         const void* k, const void* v, const void* o, const void* dout,
                         const float* lse, void* dq, void* dk, void* dv, void* workspace,
                         int64_t workspace_bytes, const RopeInv* rope,
                         const TransposedOut* tout, zk_stream_t stream);
}  // namespace zk

extern "C" int zk_attn_bwd(const zk_attn_desc* desc, const void* q,
                           const void* k, const void* v, const void* o,
                           const void* dout, const float* lse, void* dq,
                           void* dk, void* dv, void* workspace,
                           int64_t workspace_bytes, zk_stream_t stream) {
  return attn_bwd_impl("zk_attn_bwd", desc, q, k, v, o, dout, lse, dq, dk, dv, workspace,
                       workspace_bytes, nullptr, nullptr, stream);
}

namespace zk {
static int check_rope(const char* who, const zk_attn_desc* desc, const float* cos,
                      const float* sin, int64_t n_pos, const int64_t* positions, int pairing) {
  ZK_REQUIRE(cos != nullptr && sin != nullptr, ZK_EINVAL, "%s: null RoPE table", who);
  ZK_REQUIRE(pairing == ZK_ROPE_HALF || pairing == ZK_ROPE_INTERLEAVED, ZK_EINVAL,
             "%s: bad pairing %d", who, pairing);
  ZK_REQUIRE(n_pos > 0, ZK_EINVAL, "%s: empty RoPE table", who);
  ZK_REQUIRE(desc == nullptr || positions != nullptr || n_pos >= desc->Sq, ZK_EINVAL,
             "%s: table holds %lld positions < S=%lld", who, (long long)n_pos,
             (long long)(desc ? desc->Sq : 0));
  ZK_REQUIRE(desc == nullptr || desc->d % 2 == 0, ZK_EINVAL, "%s: odd head_dim", who);
  ZK_REQUIRE(aligned(cos, 16) && aligned(sin, 16), ZK_EALIGN,
             "%s: RoPE tables must be 16-byte aligned", who);
  return ZK_OK;
}
}  // namespace zk

extern "C" int zk_attn_bwd_rope_t(const zk_attn_desc* desc, const void* q, const void* k,
                                  const void* v, const void* o, const void* dout,
                                  const float* lse, void* dq, void* dk, void* dv,
                                  void* workspace, int64_t workspace_bytes, const float* cos,
                                  const float* sin, int64_t n_pos, const int64_t* positions,
                                  int pairing, void* dq_t, void* dk_t, void* dv_t, int64_t ld_t,
                                  zk_stream_t stream) {
  const char* who = "zk_attn_bwd_rope_t";
  const RopeInv r = {cos, sin, n_pos, positions, pairing};
  if (cos != nullptr || sin != nullptr) {
    const int rc = check_rope(who, desc, cos, sin, n_pos, positions, pairing);
    if (rc != ZK_OK) return rc;
  }
  const TransposedOut t = {dq_t, dk_t, dv_t, ld_t};
  return attn_bwd_impl(who, desc, q, k, v, o, dout, lse, dq, dk, dv, workspace,
                       workspace_bytes, cos != nullptr ? &r : nullptr, &t, stream);
}

extern "C" int zk_attn_bwd_rope(const zk_attn_desc* desc, const void* q, const void* k,
                                const void* v, const void* o, const void* dout,
                                const float* lse, void* dq, void* dk, void* dv,
                                void* workspace, int64_t workspace_bytes, const float* cos,
                                const float* sin, int64_t n_pos, const int64_t* positions,
                                int pairing, zk_stream_t stream) {
  const char* who = "zk_attn_bwd_rope";
  const int rc = check_rope(who, desc, cos, sin, n_pos, positions, pairing);
  if (rc != ZK_OK) return rc;
  const RopeInv r = {cos, sin, n_pos, positions, pairing};
  return attn_bwd_impl(who, desc, q, k, v, o, dout, lse, dq, dk, dv, workspace,
                       workspace_bytes, &r, nullptr, stream);
}

namespace zk {
static int attn_bwd_impl(const char* who, const zk_attn_desc* desc, const void* q,
                         const void* k, const void* v, const void* o, const void* dout,
                         const float* lse, void* dq, void* dk, void* dv, void* workspace,
                         int64_t workspace_bytes, const RopeInv* rope,
                         const TransposedOut* tout, zk_stream_t stream) {
  int rc = check_attn_desc(desc, who, true);
  if (rc != ZK_OK) return rc;
  if (tout != nullptr) {
    ZK_REQUIRE(tout->dq_t && tout->dk_t && tout->dv_t, ZK_EINVAL,
               "%s: null transposed output", who);
    ZK_REQUIRE(desc->dtype != ZK_F32, ZK_EUNSUPPORTED,
               "%s: transposed outputs need a 2-byte dtype", who);
    ZK_REQUIRE(desc->Sq % 8 == 0 && desc->Skv % 8 == 0 && tout->ld % 8 == 0 &&
                   tout->ld >= desc->B * desc->Sq && tout->ld >= desc->B * desc->Skv,
               ZK_EINVAL, "%s: transposed outputs need Sq, Skv, ld multiples of 8 and "
               "ld >= B S (ld %lld)", who, (long long)tout->ld);
    ZK_REQUIRE(aligned(tout->dq_t, 16) && aligned(tout->dk_t, 16) && aligned(tout->dv_t, 16),
               ZK_EALIGN, "%s: transposed outputs must be 16-byte aligned", who);
  }
  ZK_REQUIRE(rope == nullptr || desc->Sq == desc->Skv, ZK_EUNSUPPORTED,
             "%s: fused RoPE needs Sq == Skv", who);
  const int64_t need = zk_attn_bwd_workspace(desc);
  ZK_REQUIRE(workspace != nullptr && workspace_bytes >= need, ZK_EWORKSPACE,
             "%s: workspace %lld < %lld bytes", who,
             (long long)workspace_bytes, (long long)need);
  if (desc->B == 0 || (desc->Sq == 0 && desc->Skv == 0)) return ZK_OK;
  ZK_REQUIRE(q && k && v && o && dout && lse && dq && dk && dv, ZK_EINVAL,
             "%s: null pointer", who);
  AttnArgs a = {};
  fill_args(a, desc);
  if (rope != nullptr) {
    a.rope_cos = rope->cos;
    a.rope_sin = rope->sin;
    a.rope_npos = rope->n_pos;
    a.rope_pos = rope->positions;
    a.rope_interleaved = rope->pairing == ZK_ROPE_INTERLEAVED;
  }
  a.q = q; a.k = k; a.v = v; a.o = o; a.dout = dout; a.lse = lse;
  a.dq = dq; a.dk = dk; a.dv = dv;
  if (tout != nullptr) {
    a.dq_t = tout->dq_t;
    a.dk_t = tout->dk_t;
    a.dv_t = tout->dv_t;
    a.t_ld = tout->ld;
  }
  const uintptr_t base = (reinterpret_cast<uintptr_t>(workspace) + 255) & ~uintptr_t(255);
  a.delta = reinterpret_cast<float*>(base);
  a.lse2 = a.delta + ((desc->B * desc->Hq * desc->Sq + 63) & ~int64_t(63));
  hipStream_t s = as_stream(stream);

  const int64_t rows = desc->B * desc->Sq * desc->Hq;
  const dim3 pgrid(static_cast<unsigned>((rows * 8 + 255) / 256));
  if (desc->dtype == ZK_F32) {
    if (rows > 0) hipLaunchKernelGGL(attn_bwd_prep<float>, pgrid, dim3(256), 0, s, a);
    const int64_t qrows = desc->B * desc->Hq * desc->Sq;
    const int64_t krows = desc->B * desc->Hkv * desc->Skv;
    if (desc->d <= 64) {
      if (qrows > 0) hipLaunchKernelGGL(attn_bwd_dq_f32<64>, dim3((qrows + 63) / 64), dim3(64), 0, s, a);
      if (krows > 0) hipLaunchKernelGGL(attn_bwd_dkv_f32<64>, dim3((krows + 63) / 64), dim3(64), 0, s, a);
    } else {
      if (qrows > 0) hipLaunchKernelGGL(attn_bwd_dq_f32<128>, dim3((qrows + 63) / 64), dim3(64), 0, s, a);
      if (krows > 0) hipLaunchKernelGGL(attn_bwd_dkv_f32<128>, dim3((krows + 63) / 64), dim3(64), 0, s, a);
    }
    return launch_status(who);
  }
  ZK_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(o, 16) &&
                 aligned(dout, 16) && aligned(dq, 8) && aligned(dk, 8) && aligned(dv, 8),
             ZK_EALIGN, "%s: tensors must be 16-byte aligned", who);
  const int64_t n_kt = (desc->Skv + DkdvCfg<128>::BK - 1) / DkdvCfg<128>::BK;
  const dim3 kgrid(static_cast<unsigned>(n_kt * desc->B * desc->Hkv));
  const bool q_full = desc->Sq % DkdvCfg<128>::MQ == 0;
  const bool k_full = desc->Skv % DqCfg<128>::BN == 0;
#define ZK_BWD(T, D)                                                                        \
  do {                                                                                      \
    constexpr int BMq = DqCfg<D>::BM, NTq = DqCfg<D>::NT;                                   \
    const int64_t n_qt = (desc->Sq + BMq - 1) / BMq;                                        \
    const dim3 qgrid(static_cast<unsigned>(n_qt * desc->B * desc->Hq));                     \
    if (n_qt > 0) {                                                                         \
      if (k_full)                                                                           \
        hipLaunchKernelGGL((attn_bwd_dq<T, D, true>), qgrid, dim3(NTq), 0, s, a, n_qt);     \
      else                                                                                  \
        hipLaunchKernelGGL((attn_bwd_dq<T, D, false>), qgrid, dim3(NTq), 0, s, a, n_qt);    \
    }                                                                                       \
    if (n_kt > 0) {                                                                         \
      if (q_full)                                                                           \
        hipLaunchKernelGGL((attn_bwd_dkdv<T, D, true>), kgrid, dim3(256), 0, s, a);         \
      else                                                                                  \
        hipLaunchKernelGGL((attn_bwd_dkdv<T, D, false>), kgrid, dim3(256), 0, s, a);        \
    }                                                                                       \
  } while (0)
  if (desc->dtype == ZK_BF16) {
    if (desc->d == 128) ZK_BWD(bf16, 128); else ZK_BWD(bf16, 64);
  } else {
    if (desc->d == 128) ZK_BWD(f16, 128); else ZK_BWD(f16, 64);
  }
#undef ZK_BWD
  return launch_status(who);
}
}  // namespace zk
