// Flash-attention forward for gfx950 (bf16 / fp16 storage, fp32 softmax).
//
// Workgroup = 8 waves = 256 queries of one (batch, q-head) for d = 128, one
// workgroup per CU (two waves per SIMD; 4 waves / 128 queries for d = 64);
// each wave owns 32 queries whose Q rows stay in registers for the whole
// kernel.  The kernel streams 64-key tiles of K and V
// through LDS (row-major, XOR-swizzled 16-byte chunks, see tile_off) with the
// next tile's global loads in flight during the current tile's math; each
// tile feeds all eight waves.
//
// Orientation: the score tile is computed transposed, S^T = K Q^T, with
// v_mfma_f32_32x32x16 (A = K rows from LDS, B = Q from registers).  In the
// MFMA result layout lane l holds query (l mod 32) and 16 keys, so the online
// softmax row max / row sum are per-lane reductions plus one exchange between
// the two lane halves, and the rescale of the output accumulator is a
// per-lane scalar.  The output is also accumulated transposed,
// O^T += V^T P^T: the probabilities go from the score accumulators straight
// into the B operand (a fixed permutation of the 16 keys of each MFMA step)
// and V^T is read with the LDS transpose read in the matching order, so P
// never touches LDS and V is never transposed in memory.
//
// The running maximum is only moved (and O, l rescaled) when some lane's new
// maximum exceeds it by more than 2^8 in the exp2 domain: until then the
// probabilities are bounded by 256, which fp32 sums and bf16 / fp16 P hold
// exactly as well, and the result is the same after the final 1 / l.
//
// Masking: causal (key <= query), sliding window (key > query - W) and the
// ragged end of the key range; tiles entirely masked for a wave are skipped,
// tiles entirely visible skip the per-element mask.  Causal blocks are
// launched heaviest-first.
#include <type_traits>

#include "attn_common.h"

namespace zk {

static constexpr int kFwdThreads = 512;            // the most threads per workgroup

template <typename T, int D>
struct FwdCfg {
  // d = 128: 8 waves (one workgroup per CU at ~220 registers); d = 64: 4
  // waves, so that three workgroups of ~145 registers still share a CU
  static constexpr int NW = D == 128 ? 8 : 4;      // waves per workgroup
  static constexpr int NT = 64 * NW;
  static constexpr int BM = 32 * NW;               // queries per workgroup
  static constexpr int BN = 64;                    // keys per tile
};

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

// log2-domain growth of the running maximum tolerated before rescaling
static constexpr float kRescaleThreshold = 8.0f;

// kFull: Skv is a multiple of the key tile, so no tile runs past the end.
template <typename T, int D, bool kFull>
__global__ __launch_bounds__(kFwdThreads) __attribute__((amdgpu_waves_per_eu(2)))
void attn_fwd_kernel(AttnArgs a, int64_t n_qt) {
  typedef FwdCfg<T, D> C;
  typedef Mfma<T> M;
  typedef typename M::vec8 V8;
  constexpr int BM = C::BM, BN = C::BN, NT = C::NT;
  // each stage its own array: the compiler then sees that the next tile's
  // asynchronous loads do not alias this tile's reads (and adds no wait)
  __shared__ __attribute__((aligned(16))) T K0[BN * D], K1[BN * D], V0[BN * D], V1[BN * D];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int64_t nbh = a.B * a.Hq;
  const int64_t bid = blockIdx.x;
  const int64_t qt = n_qt - 1 - bid / nbh;  // heaviest (last) q tiles first
  const int64_t bh = bid % nbh;
  const int64_t b = bh / a.Hq, hq = bh % a.Hq;
  const int64_t hk = hq / (a.Hq / a.Hkv);
  const int64_t q0 = qt * BM;
  const int64_t qw0 = q0 + wave * 32;
  const int64_t my_q = qw0 + l32;

  const T* Qp = static_cast<const T*>(a.q) + b * a.q_sb + hq * a.q_sh;
  const T* Kp = static_cast<const T*>(a.k) + b * a.k_sb + hk * a.k_sh;
  const T* Vp = static_cast<const T*>(a.v) + b * a.v_sb + hk * a.v_sh;

  // Q^T operand: lane holds Q[my_q][16 ks + 8 g .. +7].
  V8 qreg[D / 16];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    if (my_q < a.Sq)
      qreg[ks] = *reinterpret_cast<const V8*>(Qp + my_q * a.q_ss + 16 * ks + 8 * g);
    else
      qreg[ks] = V8{};
  }

  int64_t kv_lo = 0, kv_hi = a.Skv;
  if (a.causal && kv_hi > q0 + BM) kv_hi = q0 + BM;
  if (a.window > 0 && q0 - a.window + 1 > kv_lo) kv_lo = q0 - a.window + 1;
  const int64_t t_lo = kv_lo / BN;
  const int64_t t_hi = kv_hi > kv_lo ? (kv_hi + BN - 1) / BN : t_lo;

  // K / V tiles double-buffered in LDS, loaded asynchronously one tile ahead
  TileLoader<T, D, BN, NT> kload, vload;
  kload.init(a.k_ss);
  vload.init(a.v_ss);
  auto issue = [&](int64_t k0, int st) {
    kload.issue(st ? K1 : K0, Kp, a.k_ss, k0, a.Skv, kFull);
    vload.issue(st ? V1 : V0, Vp, a.v_ss, k0, a.Skv, kFull);
  };
  // LDS byte offsets from two per-lane bases (the swizzle XORs chunk indices,
  // and a row's chunk bits never overlap its row bits): K row l32 + 32 tt,
  // chunk 2 ks + g at (rbase ^ (ks << 5)) + tt rows; the transposed V reads
  // of 32-column block nt, keys 16 kk + 4 g .. at (tbase ^ (nt << 6)) + kk
  // rows and keys 16 kk + 8 + 4 g .. at that ^ 32 plus 8 rows
  const int rbase = 2 * tile_off<D>(l32, 8 * g);
  const int tbase = 2 * tile_off<D>(4 * g + ((lane & 15) >> 2), 16 * ((lane >> 4) & 1) + 4 * (lane & 3));

  f32x16 o[D / 32];
#pragma unroll
  for (int nt = 0; nt < D / 32; ++nt) o[nt] = f32x16{};
  float m_ref = -INFINITY, l_i = 0.f;
  const float c2 = a.scale_log2;
  // Visible keys of this lane's query form one range [vis_lo, vis_lo + vis_span]
  // (causal: up to the query; window: the W keys ending at the query; always
  // below Skv), so the element mask is one unsigned compare per score.
  int vis_lo, vis_span;
  {
    const int iq = static_cast<int>(my_q);
    int hi = static_cast<int>(a.Skv) - 1;
    if (a.causal && iq < hi) hi = iq;
    const int lo = a.window > 0 ? iq - static_cast<int>(a.window) + 1 : 0;
    vis_lo = lo > 0 ? lo : 0;
    vis_span = hi - vis_lo;
    if (vis_span < 0 || my_q >= a.Sq) {  // nothing visible
      vis_lo = 0x40000000;
      vis_span = 0;
    }
  }

  // One pipeline step on LDS stage ST (a compile-time constant, so every LDS
  // address is a per-lane base plus an immediate offset).
  auto step = [&](auto stage_tag, int64_t t) {
    constexpr int st = decltype(stage_tag)::value;
    const int64_t k0 = t * BN;
    wait_vmcnt<0>();  // this wave's loads of tile t have landed
    __syncthreads();  // ... and every other wave's; all are done with the other stage
    if (t + 1 < t_hi) issue(k0 + BN, st ^ 1);
    const T* Kt = st ? K1 : K0;
    const T* Vt = st ? V1 : V0;
    // opaque per-step copies: the derived addresses are recomputed in the step
    int rb = rbase, tb = tbase;
    asm volatile("" : "+v"(rb), "+v"(tb));

    // wave-uniform tile classification
    bool skip = false, need_mask = k0 + BN > a.Skv;
    const int64_t qmin = qw0, qmax = qw0 + 31;
    if (a.causal) {
      if (k0 > qmax) skip = true;
      if (k0 + BN - 1 > qmin) need_mask = true;
    }
    if (a.window > 0) {
      if (k0 + BN - 1 <= qmin - a.window) skip = true;
      if (k0 <= qmax - a.window) need_mask = true;
    }
    if (skip) return;

    // The tile body is instantiated with and without the element mask so
    // that the masking writes sit in the same straight-line block as the MFMA
    // chain producing the scores (no branch between the two).
    auto tile = [&](auto mask_tag) {
      constexpr bool kMask = decltype(mask_tag)::value;
      // S^T = K Q^T : s[tt] covers keys k0 + 32 tt .. +31
      f32x16 s[BN / 32];
#pragma unroll
      for (int tt = 0; tt < BN / 32; ++tt) {
        s[tt] = f32x16{};
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) {
          const V8 kv = *reinterpret_cast<const V8*>(reinterpret_cast<const char*>(Kt) +
                                                     (rb ^ (ks << 5)) + tt * 32 * D * 2);
          s[tt] = M::mma(kv, qreg[ks], s[tt]);
        }
      }
      if (kMask) {
        const int kb = static_cast<int>(k0) + 4 * g - vis_lo;
#pragma unroll
        for (int tt = 0; tt < BN / 32; ++tt)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int rel = kb + 32 * tt + 8 * (j >> 2) + (j & 3);
            s[tt][j] = static_cast<unsigned>(rel) <= static_cast<unsigned>(vis_span) ? s[tt][j]
                                                                                    : -INFINITY;
          }
      }
      float mloc = -INFINITY;
#pragma unroll
      for (int tt = 0; tt < BN / 32; ++tt)
#pragma unroll
        for (int j = 0; j < 16; ++j) mloc = fmaxf(mloc, s[tt][j]);
      mloc = fmaxf(mloc, other_half(mloc));
      // move the reference maximum only when it has grown past the threshold
      const bool grow = (mloc - m_ref) * c2 > kRescaleThreshold;
      if (__any(grow)) {
        const float m_new = fmaxf(m_ref, mloc);
        const float alpha = m_new == -INFINITY ? 1.f : fast_exp2((m_ref - m_new) * c2);
        m_ref = m_new;
        l_i *= alpha;
#pragma unroll
        for (int nt = 0; nt < D / 32; ++nt) o[nt] *= alpha;
      }
      const float mc = m_ref == -INFINITY ? 0.f : m_ref * c2;

      // P^T (packed per 16-key MFMA step) and row sums
      V8 pb[BN / 16];
      float lsum = 0.f;
#pragma unroll
      for (int tt = 0; tt < BN / 32; ++tt)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float p = fast_exp2(fmaf(s[tt][j], c2, -mc));
          lsum += p;
          pb[2 * tt + (j >> 3)][j & 7] = static_cast<T>(p);
        }
      l_i += lsum;

      // O^T += V^T P^T (V^T read transposed from the row-major V tile)
#pragma unroll
      for (int kk = 0; kk < BN / 16; ++kk) {
#pragma unroll
        for (int nt = 0; nt < D / 32; ++nt) {
          typedef short s16x4 __attribute__((ext_vector_type(4)));
          typedef short s16x8 __attribute__((ext_vector_type(8)));
          typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
          const char* vb = reinterpret_cast<const char*>(Vt) + kk * 16 * D * 2;
          const int off = tb ^ (nt << 6);
          const s16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb + off));
          const s16x4 x1 =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb + 8 * D * 2 + (off ^ 32)));
          const s16x8 w = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
          o[nt] = M::mma(__builtin_bit_cast(V8, w), pb[kk], o[nt]);
        }
      }
    };
    if (need_mask)
      tile(std::true_type{});
    else
      tile(std::false_type{});
  };

  if (t_lo < t_hi) issue(t_lo * BN, 0);
  for (int64_t t = t_lo; t < t_hi; t += 2) {
    step(std::integral_constant<int, 0>{}, t);
    if (t + 1 < t_hi) step(std::integral_constant<int, 1>{}, t + 1);
  }

  const float l_tot = l_i + other_half(l_i);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  // O rounded to the storage type once, so that the row store and the
  // transposed store below write the same values (the compiler may round
  // o * inv in one step, e.g. v_fma_mix for fp16, or in two)
#pragma unroll
  for (int nt = 0; nt < D / 32; ++nt)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[nt][j] = to_f32(static_cast<T>(o[nt][j] * inv));
  if (my_q < a.Sq) {
    T* Op = static_cast<T*>(a.out) + b * a.o_sb + hq * a.o_sh + my_q * a.o_ss;
#pragma unroll
    for (int nt = 0; nt < D / 32; ++nt)
#pragma unroll
      for (int a4 = 0; a4 < 4; ++a4) {
        const int d0 = 32 * nt + 8 * a4 + 4 * g;
        typedef T T4 __attribute__((ext_vector_type(4)));
        T4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = static_cast<T>(o[nt][4 * a4 + e]);
        *reinterpret_cast<T4*>(Op + d0) = w;
      }
    if (g == 0)
      a.lse_out[(b * a.Hq + hq) * a.Sq + my_q] =
          l_tot > 0.f ? m_ref * a.scale + logf(l_tot) : -INFINITY;
  }
  if (a.o_t != nullptr) {
    // O^T rows hq D .. +D-1, token columns b Sq + q0 ..: the same rounded
    // values as the row store, through an LDS tile in the K / V stages (free
    // once every wave is past its last step)
    __syncthreads();
    const int64_t left = a.Sq - q0;
    store_rows_transposed<T, D, BM, BN * D / BM>(
        o, 1.f, K0, K1, V0, V1, static_cast<T*>(a.o_t) + hq * D * a.t_ld + b * a.Sq + q0, a.t_ld,
        static_cast<int>(left < BM ? left : BM));
  }
}

// --------------------------------------------------------------------------
// fp32 path: one thread per query row, online softmax over all keys with the
// row kept in registers.  Used for fp32 layers (small shapes); no MFMA.
template <int D>
__global__ __launch_bounds__(64) void attn_fwd_f32_kernel(AttnArgs a) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
  const int64_t total = a.B * a.Hq * a.Sq;
  if (row >= total) return;
  const int64_t qi = row % a.Sq;
  const int64_t bh = row / a.Sq;
  const int64_t b = bh / a.Hq, hq = bh % a.Hq;
  const int64_t hk = hq / (a.Hq / a.Hkv);
  const float* Q = static_cast<const float*>(a.q) + b * a.q_sb + hq * a.q_sh + qi * a.q_ss;
  const float* K = static_cast<const float*>(a.k) + b * a.k_sb + hk * a.k_sh;
  const float* V = static_cast<const float*>(a.v) + b * a.v_sb + hk * a.v_sh;
  float q[D], acc[D];
  for (int e = 0; e < D; ++e) { q[e] = e < a.d ? Q[e] : 0.f; acc[e] = 0.f; }
  float m = -INFINITY, l = 0.f;
  for (int64_t j = 0; j < a.Skv; ++j) {
    if (!attn_visible(qi, j, a.Skv, a.causal, a.window)) continue;
    const float* kr = K + j * a.k_ss;
    float s = 0.f;
    for (int e = 0; e < a.d; ++e) s = fmaf(q[e], kr[e], s);
    s *= a.scale;
    const float m_new = fmaxf(m, s);
    const float alpha = expf(m - m_new);
    const float p = expf(s - m_new);
    l = l * alpha + p;
    const float* vr = V + j * a.v_ss;
    for (int e = 0; e < a.d; ++e) acc[e] = fmaf(acc[e], alpha, p * vr[e]);
    m = m_new;
  }
  float* O = static_cast<float*>(a.out) + b * a.o_sb + hq * a.o_sh + qi * a.o_ss;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  for (int e = 0; e < a.d; ++e) O[e] = acc[e] * inv;
  a.lse_out[(b * a.Hq + hq) * a.Sq + qi] = l > 0.f ? m + logf(l) : -INFINITY;
}

}  // namespace zk

using namespace zk;

namespace zk {
// Validates a descriptor; shared by forward and backward entry points.
int check_attn_desc(const zk_attn_desc* d, const char* who, bool bwd) {
  ZK_REQUIRE(d != nullptr, ZK_EINVAL, "%s: null descriptor", who);
  ZK_REQUIRE(d->dtype == ZK_BF16 || d->dtype == ZK_F16 || d->dtype == ZK_F32,
             ZK_EDTYPE, "%s: bad dtype %d", who, d->dtype);
  ZK_REQUIRE(d->B >= 0 && d->Sq >= 0 && d->Skv >= 0 && d->Hq > 0 && d->Hkv > 0,
             ZK_EINVAL, "%s: bad shape", who);
  ZK_REQUIRE(d->Hq % d->Hkv == 0, ZK_EINVAL,
             "%s: Hq=%lld not a multiple of Hkv=%lld", who, (long long)d->Hq,
             (long long)d->Hkv);
  ZK_REQUIRE(d->window >= 0, ZK_EINVAL, "%s: negative window", who);
  ZK_REQUIRE(!(d->causal || d->window > 0) || d->Sq == d->Skv, ZK_EUNSUPPORTED,
             "%s: masked attention needs Sq == Skv (got %lld, %lld)", who,
             (long long)d->Sq, (long long)d->Skv);
  if (d->dtype == ZK_F32) {
    ZK_REQUIRE(d->d > 0 && d->d <= 128, ZK_EUNSUPPORTED,
               "%s: fp32 path supports head_dim <= 128 (got %lld)", who,
               (long long)d->d);
  } else {
    ZK_REQUIRE(d->d == 64 || d->d == 128, ZK_EUNSUPPORTED,
               "%s: head_dim must be 64 or 128 (got %lld)", who, (long long)d->d);
    // 16-byte vector access along d and along rows
    const int64_t strides[] = {d->q_sb, d->q_ss, d->q_sh, d->k_sb, d->k_ss,
                               d->k_sh, d->v_sb, d->v_ss, d->v_sh, d->o_sb,
                               d->o_ss, d->o_sh};
    for (int64_t s : strides)
      ZK_REQUIRE(s % 8 == 0, ZK_EALIGN,
                 "%s: strides must be multiples of 8 elements (got %lld)", who,
                 (long long)s);
    if (bwd) {
      const int64_t bs[] = {d->dq_sb, d->dq_ss, d->dq_sh, d->dk_sb, d->dk_ss,
                            d->dk_sh, d->dv_sb, d->dv_ss, d->dv_sh};
      for (int64_t s : bs)
        ZK_REQUIRE(s % 8 == 0, ZK_EALIGN,
                   "%s: grad strides must be multiples of 8 elements", who);
    }
    // the tile loaders keep a 32-row span of one tensor in a 32-bit byte offset
    const int64_t rs[] = {d->q_ss, d->k_ss, d->v_ss, d->o_ss};
    for (int64_t s : rs)
      ZK_REQUIRE(s >= 0 && s < (int64_t(1) << 26), ZK_EUNSUPPORTED,
                 "%s: row stride %lld out of range", who, (long long)s);
  }
  ZK_REQUIRE(d->B * d->Hq * ((d->Sq + 127) / 128) < 0x7fffffffLL, ZK_EINVAL,
             "%s: grid too large", who);
  return ZK_OK;
}

void fill_args(AttnArgs& a, const zk_attn_desc* d) {
  a.B = d->B; a.Sq = d->Sq; a.Skv = d->Skv; a.Hq = d->Hq; a.Hkv = d->Hkv; a.d = d->d;
  a.q_sb = d->q_sb; a.q_ss = d->q_ss; a.q_sh = d->q_sh;
  a.k_sb = d->k_sb; a.k_ss = d->k_ss; a.k_sh = d->k_sh;
  a.v_sb = d->v_sb; a.v_ss = d->v_ss; a.v_sh = d->v_sh;
  a.o_sb = d->o_sb; a.o_ss = d->o_ss; a.o_sh = d->o_sh;
  a.dq_sb = d->dq_sb; a.dq_ss = d->dq_ss; a.dq_sh = d->dq_sh;
  a.dk_sb = d->dk_sb; a.dk_ss = d->dk_ss; a.dk_sh = d->dk_sh;
  a.dv_sb = d->dv_sb; a.dv_ss = d->dv_ss; a.dv_sh = d->dv_sh;
  a.scale = d->scale;
  a.scale_log2 = d->scale * kLog2e;
  a.causal = d->causal;
  a.window = d->window;
}
}  // namespace zk

static int attn_fwd_impl(const char* who, const zk_attn_desc* desc, const void* q,
                         const void* k, const void* v, void* o, float* lse, void* o_t,
                         int64_t ld_t, zk_stream_t stream) {
  int rc = check_attn_desc(desc, who, false);
  if (rc != ZK_OK) return rc;
  if (o_t != nullptr) {
    ZK_REQUIRE(desc->dtype != ZK_F32, ZK_EUNSUPPORTED,
               "%s: the transposed output needs a 2-byte dtype", who);
    ZK_REQUIRE(desc->Sq % 8 == 0 && ld_t % 8 == 0 && ld_t >= desc->B * desc->Sq, ZK_EINVAL,
               "%s: the transposed output needs Sq, ld multiples of 8 and ld >= B Sq (ld %lld)",
               who, (long long)ld_t);
    ZK_REQUIRE(aligned(o_t, 16), ZK_EALIGN, "%s: the transposed output must be 16-byte aligned",
               who);
  }
  if (desc->B == 0 || desc->Sq == 0) return ZK_OK;
  ZK_REQUIRE(q && k && v && o && lse, ZK_EINVAL, "%s: null pointer", who);
  AttnArgs a = {};
  fill_args(a, desc);
  a.q = q; a.k = k; a.v = v; a.out = o; a.lse_out = lse;
  a.o_t = o_t;
  a.t_ld = ld_t;
  hipStream_t s = as_stream(stream);
  if (desc->dtype == ZK_F32) {
    const int64_t rows = desc->B * desc->Hq * desc->Sq;
    const dim3 grid(static_cast<unsigned>((rows + 63) / 64));
    if (desc->d <= 64)
      hipLaunchKernelGGL(attn_fwd_f32_kernel<64>, grid, dim3(64), 0, s, a);
    else
      hipLaunchKernelGGL(attn_fwd_f32_kernel<128>, grid, dim3(64), 0, s, a);
    return launch_status(who);
  }
  ZK_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(o, 16),
             ZK_EALIGN, "%s: q/k/v/o must be 16-byte aligned", who);
#define ZK_FWD(T, D)                                                                    \
  do {                                                                                  \
    constexpr int BM = FwdCfg<T, D>::BM, NT = FwdCfg<T, D>::NT;                         \
    const int64_t n_qt = (desc->Sq + BM - 1) / BM;                                      \
    const dim3 grid(static_cast<unsigned>(n_qt * desc->B * desc->Hq));                  \
    if (desc->Skv % FwdCfg<T, D>::BN == 0)                                              \
      hipLaunchKernelGGL((attn_fwd_kernel<T, D, true>), grid, dim3(NT), 0, s, a, n_qt);    \
    else                                                                                \
      hipLaunchKernelGGL((attn_fwd_kernel<T, D, false>), grid, dim3(NT), 0, s, a, n_qt);  \
  } while (0)
  if (desc->dtype == ZK_BF16) {
    if (desc->d == 128) ZK_FWD(bf16, 128); else ZK_FWD(bf16, 64);
  } else {
    if (desc->d == 128) ZK_FWD(f16, 128); else ZK_FWD(f16, 64);
  }
#undef ZK_FWD
  return launch_status(who);
}

extern "C" int zk_attn_fwd(const zk_attn_desc* desc, const void* q, const void* k, const void* v,
                           void* o, float* lse, zk_stream_t stream) {
  return attn_fwd_impl("zk_attn_fwd", desc, q, k, v, o, lse, nullptr, 0, stream);
}

extern "C" int zk_attn_fwd_t(const zk_attn_desc* desc, const void* q, const void* k,
                             const void* v, void* o, float* lse, void* o_t, int64_t ld_t,
                             zk_stream_t stream) {
  ZK_REQUIRE(o_t != nullptr, ZK_EINVAL, "zk_attn_fwd_t: null transposed output");
  return attn_fwd_impl("zk_attn_fwd_t", desc, q, k, v, o, lse, o_t, ld_t, stream);
}
