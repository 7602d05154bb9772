// Flash-attention backward for gfx950 (bf16 / fp16 storage).
//
// Three kernels:
//  1. attn_bwd_prep: delta[b,h,i] = sum_d dO[i,d] * O[i,d] (fp32) and zeroes
//     the fp32 dQ accumulator rows it visits (no memset node, so the whole
//     backward can be captured in a graph).
//  2. attn_bwd_kernel: KV-stationary.  A workgroup owns 128 keys of one
//     (batch, kv-head) -- 32 keys per wave, with that wave's K and V rows held
//     in registers as MFMA operands -- and loops over every 32-query block of
//     every q-head in the GQA group (the group reduction of dK / dV happens in
//     registers, repeat_kv is never materialised).  Per query block:
//       S   = Q K^T          (A = Q from LDS, B = K from registers)
//       P   = exp2(S*scale*log2e - lse*log2e), masked
//       dP  = dO V^T         (A = dO from LDS, B = V from registers)
//       dS  = P (dP - delta)
//       dV^T += dO^T P,  dK^T += Q^T dS   (P / dS feed the B operand straight
//                          from the score accumulators; Q^T / dO^T from LDS)
//       dQ  += dS K          (dS and the workgroup's K^T through LDS),
//                          added into the fp32 accumulator with hardware
//                          fp32 atomics, one row-contiguous store per lane.
//     dK and dV are written once at the end (scaled), rounded to storage type.
//  3. attn_bwd_dq_store: dq = round(dq_acc).
#include "attn_common.h"

namespace zk {

int check_attn_desc(const zk_attn_desc* d, const char* who, bool bwd);
void fill_args(AttnArgs& a, const zk_attn_desc* d);

// ----------------------------------------------------------------- prep ----
// 8 lanes per (b, q, h) row; each lane covers d/8 elements.
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
    float* acc_row = a.dq_acc + row * a.d;
    for (int64_t e = sub; e < a.d; e += 8) {
      acc = fmaf(to_f32(Or[e]), to_f32(Dr[e]), acc);
      acc_row[e] = 0.f;
    }
  }
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  acc += __shfl_xor(acc, 4, 64);
  if (row < rows && sub == 0) a.delta[(b * a.Hq + h) * a.Sq + q] = acc;
}

// ------------------------------------------------------------ dq store -----
template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_dq_store(AttnArgs a) {
  const int64_t total = a.B * a.Sq * a.Hq * a.d;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
       i < total; i += stride) {
    const int64_t e = i % a.d;
    int64_t r = i / a.d;
    const int64_t h = r % a.Hq; r /= a.Hq;
    const int64_t q = r % a.Sq;
    const int64_t b = r / a.Sq;
    T* dq = static_cast<T*>(a.dq);
    dq[b * a.dq_sb + q * a.dq_ss + h * a.dq_sh + e] = from_f32<T>(a.dq_acc[i]);
  }
}

// -------------------------------------------------------------- main -------
template <int D>
struct BwdCfg {
  static constexpr int BK = 128;       // keys per workgroup (32 per wave)
  static constexpr int MQ = 32;        // queries per iteration
  static constexpr int QP = D + 8;     // row-major Q / dO pitch (elements)
  static constexpr int TP = MQ + 4;    // transposed Q^T / dO^T pitch
  static constexpr int SP = BK + 8;    // dS pitch
  static constexpr int NSL = D / 32;   // d slices of 32 for dQ
  static constexpr int KSPLIT = 4 / NSL;            // key groups for dQ
  static constexpr int KGK = BK / KSPLIT;           // keys per dQ group
  static constexpr int UNITS = (MQ / 2) * (D / 8);  // (row pair, 8-col chunk)
  static_assert(NSL * KSPLIT == 4, "d must be 64 or 128");
  static_assert(UNITS <= 256, "tile too large");
};

template <typename T, int D>
__global__ __launch_bounds__(256) void attn_bwd_kernel(AttnArgs a, int64_t n_kt) {
  typedef BwdCfg<D> C;
  typedef Mfma<T> M;
  typedef typename M::vec8 V8;
  constexpr int BK = C::BK, MQ = C::MQ, QP = C::QP, TP = C::TP, SP = C::SP;
  __shared__ __attribute__((aligned(16))) T Qs[MQ * QP];
  __shared__ __attribute__((aligned(16))) T dOs[MQ * QP];
  __shared__ __attribute__((aligned(16))) T Qt[D * TP];
  __shared__ __attribute__((aligned(16))) T dOt[D * TP];
  __shared__ __attribute__((aligned(16))) T dSs[MQ * SP];
  __shared__ __attribute__((aligned(16))) T Kt[D * SP];
  __shared__ __attribute__((aligned(16))) float lse2s[MQ];
  __shared__ __attribute__((aligned(16))) float dels[MQ];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int64_t nbh = a.B * a.Hkv;
  const int64_t bid = blockIdx.x;
  const int64_t kt = bid / nbh;  // low key tiles carry the most causal work
  const int64_t bh = bid % nbh;
  const int64_t b = bh / a.Hkv, hk = bh % a.Hkv;
  const int64_t n_rep = a.Hq / a.Hkv;
  const int64_t k0 = kt * BK;
  const int64_t kw0 = k0 + 32 * wave;
  const int64_t my_key = kw0 + l32;
  const float c2 = a.scale_log2;

  const T* Kp = static_cast<const T*>(a.k) + b * a.k_sb + hk * a.k_sh;
  const T* Vp = static_cast<const T*>(a.v) + b * a.v_sb + hk * a.v_sh;

  // B operands for S = Q K^T and dP = dO V^T: lane holds row my_key.
  V8 kreg[D / 16], vreg[D / 16];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    if (my_key < a.Skv) {
      kreg[ks] = *reinterpret_cast<const V8*>(Kp + my_key * a.k_ss + 16 * ks + 8 * g);
      vreg[ks] = *reinterpret_cast<const V8*>(Vp + my_key * a.v_ss + 16 * ks + 8 * g);
    } else {
      kreg[ks] = V8{};
      vreg[ks] = V8{};
    }
  }
  // B operand for dQ = dS K, read from Kt[dsl + l32][kbase + 16 kk + 8 g ..]:
  // K^T of the workgroup's keys, written once (key pairs packed per 32-bit).
  const int dsl = 32 * (wave % C::NSL);
  const int kbase = C::KGK * (wave / C::NSL);
  for (int u = tid; u < (BK / 2) * (D / 8); u += 256) {
    const int kp = u % (BK / 2), dch = u / (BK / 2);
    const int64_t key = k0 + 2 * kp;
    const uint4 r0 = key < a.Skv ? *reinterpret_cast<const uint4*>(Kp + key * a.k_ss + dch * 8)
                                 : make_uint4(0, 0, 0, 0);
    const uint4 r1 = key + 1 < a.Skv
                         ? *reinterpret_cast<const uint4*>(Kp + (key + 1) * a.k_ss + dch * 8)
                         : make_uint4(0, 0, 0, 0);
    const uint16_t* e0 = reinterpret_cast<const uint16_t*>(&r0);
    const uint16_t* e1 = reinterpret_cast<const uint16_t*>(&r1);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      *reinterpret_cast<uint32_t*>(&Kt[(dch * 8 + e) * SP + 2 * kp]) =
          static_cast<uint32_t>(e0[e]) | (static_cast<uint32_t>(e1[e]) << 16);
  }

  f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
  for (int nt = 0; nt < D / 32; ++nt) {
    dk[nt] = f32x16{};
    dv[nt] = f32x16{};
  }

  // query range that can see keys [k0, k0 + BK)
  int64_t q_lo = 0, q_hi = a.Sq;
  if (a.causal) q_lo = k0;
  if (a.window > 0 && k0 + BK - 1 + a.window < q_hi) q_hi = k0 + BK - 1 + a.window;
  const int64_t qb_lo = q_lo / MQ;
  const int64_t qb_hi = q_hi > q_lo ? (q_hi + MQ - 1) / MQ : qb_lo;
  const int64_t nqb = qb_hi - qb_lo;
  const int64_t n_iter = nqb * n_rep;

  // staging registers for the next (head, query block)
  uint4 qr[2], dr[2];
  float lse_r = 0.f, del_r = 0.f;
  const bool loader = tid < C::UNITS;
  const int up = tid % (MQ / 2), udch = tid / (MQ / 2);
  auto prefetch = [&](int64_t it) {
    const int64_t hq = hk * n_rep + it / nqb;
    const int64_t qb0 = (qb_lo + it % nqb) * MQ;
    if (loader) {
      const T* Qp = static_cast<const T*>(a.q) + b * a.q_sb + hq * a.q_sh;
      const T* Dp = static_cast<const T*>(a.dout) + b * a.o_sb + hq * a.o_sh;
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int64_t qi = qb0 + 2 * up + r;
        if (qi < a.Sq) {
          qr[r] = *reinterpret_cast<const uint4*>(Qp + qi * a.q_ss + udch * 8);
          dr[r] = *reinterpret_cast<const uint4*>(Dp + qi * a.o_ss + udch * 8);
        } else {
          qr[r] = make_uint4(0, 0, 0, 0);
          dr[r] = make_uint4(0, 0, 0, 0);
        }
      }
    }
    if (tid < MQ) {
      const int64_t qi = qb0 + tid;
      if (qi < a.Sq) {
        const float l = a.lse[(b * a.Hq + hq) * a.Sq + qi];
        lse_r = l == -INFINITY ? INFINITY : l * kLog2e;
        del_r = a.delta[(b * a.Hq + hq) * a.Sq + qi];
      } else {
        lse_r = INFINITY;  // P = 0 for rows past the end
        del_r = 0.f;
      }
    }
  };
  auto store_lds = [&]() {
    if (loader) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        *reinterpret_cast<uint4*>(&Qs[(2 * up + r) * QP + udch * 8]) = qr[r];
        *reinterpret_cast<uint4*>(&dOs[(2 * up + r) * QP + udch * 8]) = dr[r];
      }
      const uint16_t* q0e = reinterpret_cast<const uint16_t*>(&qr[0]);
      const uint16_t* q1e = reinterpret_cast<const uint16_t*>(&qr[1]);
      const uint16_t* d0e = reinterpret_cast<const uint16_t*>(&dr[0]);
      const uint16_t* d1e = reinterpret_cast<const uint16_t*>(&dr[1]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int row = udch * 8 + e;
        *reinterpret_cast<uint32_t*>(&Qt[row * TP + 2 * up]) =
            static_cast<uint32_t>(q0e[e]) | (static_cast<uint32_t>(q1e[e]) << 16);
        *reinterpret_cast<uint32_t*>(&dOt[row * TP + 2 * up]) =
            static_cast<uint32_t>(d0e[e]) | (static_cast<uint32_t>(d1e[e]) << 16);
      }
    }
    if (tid < MQ) {
      lse2s[tid] = lse_r;
      dels[tid] = del_r;
    }
  };

  if (n_iter > 0) prefetch(0);
  for (int64_t it = 0; it < n_iter; ++it) {
    const int64_t hq = hk * n_rep + it / nqb;
    const int64_t qb0 = (qb_lo + it % nqb) * MQ;
    __syncthreads();
    store_lds();
    __syncthreads();
    if (it + 1 < n_iter) prefetch(it + 1);

    bool skip = false, need_mask = kw0 + 31 >= a.Skv;
    if (a.causal) {
      if (kw0 > qb0 + MQ - 1) skip = true;
      if (kw0 + 31 > qb0) need_mask = true;
    }
    if (a.window > 0) {
      if (kw0 + 31 <= qb0 - a.window) skip = true;
      if (kw0 <= qb0 + MQ - 1 - a.window) need_mask = true;
    }

    if (!skip) {
      // S = Q K^T and dP = dO V^T (rows = queries, cols = this wave's keys)
      f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
        const V8 qa = *reinterpret_cast<const V8*>(&Qs[l32 * QP + 16 * ks + 8 * g]);
        s = M::mma(qa, kreg[ks], s);
        const V8 da = *reinterpret_cast<const V8*>(&dOs[l32 * QP + 16 * ks + 8 * g]);
        dp = M::mma(da, vreg[ks], dp);
      }
      V8 pb[2], sb[2];
#pragma unroll
      for (int a4 = 0; a4 < 4; ++a4) {
        const float4 l4 = *reinterpret_cast<const float4*>(&lse2s[8 * a4 + 4 * g]);
        const float4 d4 = *reinterpret_cast<const float4*>(&dels[8 * a4 + 4 * g]);
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
        const float dl[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = 4 * a4 + e;
          float p = __builtin_amdgcn_exp2f(fmaf(s[j], c2, -lv[e]));
          if (need_mask) {
            const int64_t qi = qb0 + 8 * a4 + 4 * g + e;
            if (!attn_visible(qi, my_key, a.Skv, a.causal, a.window)) p = 0.f;
          }
          const float ds = p * (dp[j] - dl[e]);
          pb[j >> 3][j & 7] = static_cast<T>(p);
          sb[j >> 3][j & 7] = static_cast<T>(ds);
          dSs[(8 * a4 + 4 * g + e) * SP + 32 * wave + l32] = static_cast<T>(ds);
        }
      }
      // dV^T += dO^T P ; dK^T += Q^T dS
#pragma unroll
      for (int nt = 0; nt < D / 32; ++nt) {
        const T* drow = &dOt[(32 * nt + l32) * TP];
        const T* qrow = &Qt[(32 * nt + l32) * TP];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const int qb = 16 * kk + 4 * g;
          const u32x2 dlo = *reinterpret_cast<const u32x2*>(drow + qb);
          const u32x2 dhi = *reinterpret_cast<const u32x2*>(drow + qb + 8);
          const u32x4 dw = {dlo[0], dlo[1], dhi[0], dhi[1]};
          dv[nt] = M::mma(__builtin_bit_cast(V8, dw), pb[kk], dv[nt]);
          const u32x2 qlo = *reinterpret_cast<const u32x2*>(qrow + qb);
          const u32x2 qhi = *reinterpret_cast<const u32x2*>(qrow + qb + 8);
          const u32x4 qw = {qlo[0], qlo[1], qhi[0], qhi[1]};
          dk[nt] = M::mma(__builtin_bit_cast(V8, qw), sb[kk], dk[nt]);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j)
        dSs[(8 * (j >> 2) + 4 * g + (j & 3)) * SP + 32 * wave + l32] = static_cast<T>(0.f);
    }
    __syncthreads();

    // dQ[:, dsl..dsl+31] += dS[:, kbase..kbase+KGK) K[kbase.., dsl..]
    f32x16 dq = f32x16{};
#pragma unroll
    for (int kk = 0; kk < C::KGK / 16; ++kk) {
      const V8 sa = *reinterpret_cast<const V8*>(&dSs[l32 * SP + kbase + 16 * kk + 8 * g]);
      const V8 kb = *reinterpret_cast<const V8*>(&Kt[(dsl + l32) * SP + kbase + 16 * kk + 8 * g]);
      dq = M::mma(sa, kb, dq);
    }
    float* accp = a.dq_acc + ((b * a.Sq + qb0) * a.Hq + hq) * D + dsl + l32;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int qrow = 8 * (j >> 2) + 4 * g + (j & 3);
      if (qb0 + qrow < a.Sq)
        unsafeAtomicAdd(accp + static_cast<int64_t>(qrow) * a.Hq * D, dq[j] * a.scale);
    }
  }

  // dK = scale * (Q^T dS)^T, dV = (dO^T P)^T : lane holds key my_key and
  // d rows 32 nt + 8 a4 + 4 g + 0..3 (4 consecutive elements).
  if (my_key < a.Skv) {
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
}

// ------------------------------------------------------------- fp32 path ---
// Simple per-row kernels for fp32 layers (small shapes, no MFMA).
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
  float* dkp = static_cast<float*>(a.dk) + b * a.dk_sb + hk * a.dk_sh + kj * a.dk_ss;
  float* dvp = static_cast<float*>(a.dv) + b * a.dv_sb + hk * a.dv_sh + kj * a.dv_ss;
  for (int e = 0; e < a.d; ++e) { dkp[e] = dk[e]; dvp[e] = dv[e]; }
}

}  // namespace zk

using namespace zk;

extern "C" int64_t zk_attn_bwd_workspace(const zk_attn_desc* desc) {
  if (desc == nullptr) return 0;
  const int64_t acc = desc->B * desc->Sq * desc->Hq * desc->d;  // fp32 dQ
  const int64_t del = desc->B * desc->Hq * desc->Sq;            // fp32 delta
  return (acc + del) * 4 + 256;
}

extern "C" int zk_attn_bwd(const zk_attn_desc* desc, const void* q,
                           const void* k, const void* v, const void* o,
                           const void* dout, const float* lse, void* dq,
                           void* dk, void* dv, void* workspace,
                           int64_t workspace_bytes, zk_stream_t stream) {
  int rc = check_attn_desc(desc, "zk_attn_bwd", true);
  if (rc != ZK_OK) return rc;
  const int64_t need = zk_attn_bwd_workspace(desc);
  ZK_REQUIRE(workspace != nullptr && workspace_bytes >= need, ZK_EWORKSPACE,
             "zk_attn_bwd: workspace %lld < %lld bytes",
             (long long)workspace_bytes, (long long)need);
  if (desc->B == 0 || (desc->Sq == 0 && desc->Skv == 0)) return ZK_OK;
  ZK_REQUIRE(q && k && v && o && dout && lse && dq && dk && dv, ZK_EINVAL,
             "zk_attn_bwd: null pointer");
  AttnArgs a = {};
  fill_args(a, desc);
  a.q = q; a.k = k; a.v = v; a.o = o; a.dout = dout; a.lse = lse;
  a.dq = dq; a.dk = dk; a.dv = dv;
  const uintptr_t base = (reinterpret_cast<uintptr_t>(workspace) + 255) & ~uintptr_t(255);
  a.dq_acc = reinterpret_cast<float*>(base);
  a.delta = a.dq_acc + desc->B * desc->Sq * desc->Hq * desc->d;
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
    return launch_status("zk_attn_bwd");
  }
  ZK_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(o, 16) &&
                 aligned(dout, 16) && aligned(dk, 8) && aligned(dv, 8),
             ZK_EALIGN, "zk_attn_bwd: tensors must be 16-byte aligned");
  const int64_t n_kt = (desc->Skv + 127) / 128;
  const dim3 grid(static_cast<unsigned>(n_kt * desc->B * desc->Hkv));
  int64_t sgrid = (rows * desc->d + 255) / 256;
  const int64_t cap = static_cast<int64_t>(device_cus()) * 16;
  if (sgrid > cap) sgrid = cap;
#define ZK_BWD(T, D)                                                              \
  do {                                                                            \
    if (rows > 0) hipLaunchKernelGGL(attn_bwd_prep<T>, pgrid, dim3(256), 0, s, a); \
    if (n_kt > 0) hipLaunchKernelGGL((attn_bwd_kernel<T, D>), grid, dim3(256), 0, s, a, n_kt); \
    if (rows > 0) hipLaunchKernelGGL(attn_bwd_dq_store<T>, dim3(sgrid), dim3(256), 0, s, a); \
  } while (0)
  if (desc->dtype == ZK_BF16) {
    if (desc->d == 128) ZK_BWD(bf16, 128); else ZK_BWD(bf16, 64);
  } else {
    if (desc->d == 128) ZK_BWD(f16, 128); else ZK_BWD(f16, 64);
  }
#undef ZK_BWD
  return launch_status("zk_attn_bwd");
}
