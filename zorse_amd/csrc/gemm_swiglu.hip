// gate|up projection GEMM with the SwiGLU epilogue (gfx950, bf16 / fp16).
//
//   g = x Wg^T,  u = x Wu^T           (fp32 accumulation, rounded to T)
//   z = round(round(silu(g)) * u)     (the LlamaMLP activation, same rounding
//                                      points as the unfused GEMM + SwiGLU)
// x [M, K] and the weights [F, K] are row-major with K contiguous (the
// nn.Linear layout), so both MFMA operands stream along the reduction.
//
// Workgroup = 4 waves, tile = 128 tokens x 64 features of both g and u; the
// B tile holds the 64 gate rows followed by the 64 up rows of the same
// features, so every lane ends with g and u of the same (token, feature) and
// the activation is computed in registers.  Waves split the tile 2 x 2: 64
// tokens x 32 features, i.e. two 32-row MFMA blocks for each of g and u
// (v_mfma_f32_32x32x16, A = x rows, B = weight rows, both read as 16-byte
// rows of XOR-swizzled LDS tiles).  K advances in steps of 64 through two
// LDS stages filled by asynchronous global->LDS loads one step ahead (the
// stages are separate arrays so that the compiler sees the loads into one do
// not alias reads of the other).  The epilogue stages g, u, z through the
// then idle LDS (same swizzle) and writes 16-byte row chunks; the optional
// transposed copy z^T [F, M] (for down_proj's weight gradient) is written
// from the same staged tile.  Workgroups are ordered in groups of 16 token
// tiles per feature tile so that the blocks running together share their x
// and weight rows in the caches.
#include "attn_common.h"
#include "vec.h"

namespace zk {

struct GemmSwigluCfg {
  static constexpr int BM = 128;  // tokens per workgroup
  static constexpr int BF = 64;   // features per workgroup (g and u each)
  static constexpr int BK = 64;   // reduction step
  static constexpr int GROUP_M = 16;
};

template <typename T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void gemm_swiglu_kernel(const T* __restrict__ x, int64_t ld_x, const T* __restrict__ wg,
                        const T* __restrict__ wu, int64_t ld_w, T* __restrict__ g_out,
                        T* __restrict__ u_out, int64_t ld_gu, T* __restrict__ z,
                        int64_t ld_z, T* __restrict__ zt, int64_t ld_zt, int64_t M,
                        int64_t F, int64_t K) {
  typedef GemmSwigluCfg C;
  typedef Mfma<T> Mm;
  typedef typename Mm::vec8 V8;
  constexpr int BM = C::BM, BF = C::BF, BK = C::BK;
  __shared__ __attribute__((aligned(16))) T As0[BM * BK];
  __shared__ __attribute__((aligned(16))) T As1[BM * BK];
  __shared__ __attribute__((aligned(16))) T Bs0[2 * BF * BK];
  __shared__ __attribute__((aligned(16))) T Bs1[2 * BF * BK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;  // 64-token half, 32-feature half

  // grouped order: GROUP_M token tiles per feature tile, feature tiles next
  const int64_t n_m = (M + BM - 1) / BM, n_f = (F + BF - 1) / BF;
  const int64_t pid = blockIdx.x;
  const int64_t per_group = static_cast<int64_t>(C::GROUP_M) * n_f;
  const int64_t grp = pid / per_group;
  const int64_t m_first = grp * C::GROUP_M;
  const int64_t gm = n_m - m_first < C::GROUP_M ? n_m - m_first : C::GROUP_M;
  const int64_t in_grp = pid - grp * per_group;
  const int64_t tm = m_first + in_grp % gm;
  const int64_t tf = in_grp / gm;
  const int64_t m0 = tm * BM, f0 = tf * BF;

  TileLoader<T, BK, BM> aload;
  TileLoader<T, BK, BF> bload;
  aload.init(ld_x);
  bload.init(ld_w);
  const bool a_full = m0 + BM <= M, b_full = f0 + BF <= F;
  const T* xa = x;
  auto issue = [&](int64_t k0, T* as, T* bs) __attribute__((always_inline)) {
    aload.issue(as, xa + k0, ld_x, m0, M, a_full);
    bload.issue(bs, wg + k0, ld_w, f0, F, b_full);
    bload.issue(bs + BF * BK, wu + k0, ld_w, f0, F, b_full);
  };

  f32x16 accg[2], accu[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    accg[i] = f32x16{};
    accu[i] = f32x16{};
  }

  auto step = [&](auto stage_tag, int64_t kt, int64_t n_k) __attribute__((always_inline)) {
    constexpr int st = decltype(stage_tag)::value;
    const T* as = st ? As1 : As0;
    const T* bs = st ? Bs1 : Bs0;
    wait_vmcnt<0>();  // this wave's loads of step kt have landed
    __syncthreads();  // ... and every wave's; all are done with the other stage
    if (kt + 1 < n_k) issue((kt + 1) * BK, st ? As0 : As1, st ? Bs0 : Bs1);
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      const int col = 16 * s + 8 * g;
      V8 a[2], bg, bu;
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
        a[mi] = *reinterpret_cast<const V8*>(&as[tile_off<BK>(wm * 64 + 32 * mi + l32, col)]);
      bg = *reinterpret_cast<const V8*>(&bs[tile_off<BK>(wn * 32 + l32, col)]);
      bu = *reinterpret_cast<const V8*>(&bs[tile_off<BK>(BF + wn * 32 + l32, col)]);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        accg[mi] = Mm::mma(a[mi], bg, accg[mi]);
        accu[mi] = Mm::mma(a[mi], bu, accu[mi]);
      }
    }
    // the compiler's single-wave MFMA / LDS interleaving strategy
    __builtin_amdgcn_iglp_opt(1);
  };

  const int64_t n_k = K / BK;
  issue(0, As0, Bs0);
  for (int64_t kt = 0; kt < n_k; kt += 2) {
    step(std::integral_constant<int, 0>{}, kt, n_k);
    if (kt + 1 < n_k) step(std::integral_constant<int, 1>{}, kt + 1, n_k);
  }

  // ---- epilogue: stage g, u, z (rounded to T) in the idle LDS -----------
  __syncthreads();  // every wave is done reading the last stage
  T* Gs = As0;      // [BM][BF] each, swizzled rows of 64 elements
  T* Us = As1;
  T* Zs = Bs0;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int r = wm * 64 + 32 * mi + 8 * (j >> 2) + 4 * g + (j & 3);
      const int c = wn * 32 + l32;
      const float gv = round_to<T>(accg[mi][j]);
      const float uv = round_to<T>(accu[mi][j]);
      const float sv = round_to<T>(gv / (1.0f + expf(-gv)));
      const int off = tile_off<BF>(r, c);
      Gs[off] = static_cast<T>(gv);
      Us[off] = static_cast<T>(uv);
      Zs[off] = static_cast<T>(sv * uv);
    }
  __syncthreads();
  // rows: 128 tokens x 8 chunks of 8 features, 4 chunks per thread per tensor
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = i * 256 + tid;
    const int r = q >> 3, ch = q & 7;
    const int64_t gr = m0 + r, gc = f0 + 8 * ch;
    if (gr < M && gc < F) {
      const int off = tile_off<BF>(r, 8 * ch);
      const uint4 wg8 = *reinterpret_cast<const uint4*>(&Gs[off]);
      const uint4 wu8 = *reinterpret_cast<const uint4*>(&Us[off]);
      const uint4 wz8 = *reinterpret_cast<const uint4*>(&Zs[off]);
      *reinterpret_cast<uint4*>(g_out + gr * ld_gu + gc) = wg8;
      *reinterpret_cast<uint4*>(u_out + gr * ld_gu + gc) = wu8;
      *reinterpret_cast<uint4*>(z + gr * ld_z + gc) = wz8;
    }
  }
  if (zt != nullptr) {
    // z^T rows: 64 features x 16 chunks of 8 tokens, 4 per thread
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = i * 256 + tid;
      const int c = q >> 4, rch = q & 15;
      const int64_t gc = f0 + c, gr = m0 + 8 * rch;
      if (gc < F && gr < M) {
        typedef T T8 __attribute__((ext_vector_type(8)));
        T8 w;
#pragma unroll
        for (int e = 0; e < 8; ++e) w[e] = Zs[tile_off<BF>(8 * rch + e, c)];
        *reinterpret_cast<T8*>(zt + gc * ld_zt + gr) = w;
      }
    }
  }
}

}  // namespace zk

namespace zk {
// the 256 x 256 pipeline of gemm.hip, for the shapes it takes
int zk_gemm_swiglu_tiled_supported(int64_t M, int64_t F, int64_t K);
int zk_gemm_swiglu_tiled(const void* x, int64_t ld_x, const void* w_gate, const void* w_up,
                         int64_t ld_w, void* g_out, void* u_out, int64_t ld_gu, void* z,
                         int64_t ld_z, void* zt, int64_t ld_zt, int64_t M, int64_t F, int64_t K,
                         int dtype, zk_stream_t stream);
}  // namespace zk

using namespace zk;

extern "C" int zk_gemm_swiglu(const void* x, int64_t ld_x, const void* w_gate,
                              const void* w_up, int64_t ld_w, void* g_out, void* u_out,
                              int64_t ld_gu, void* z, int64_t ld_z, void* zt, int64_t ld_zt,
                              int64_t M, int64_t F, int64_t K, int dtype, zk_stream_t stream) {
  typedef GemmSwigluCfg C;
  ZK_REQUIRE(dtype == ZK_BF16 || dtype == ZK_F16, ZK_EDTYPE,
             "zk_gemm_swiglu: 2-byte dtypes only (got %d)", dtype);
  ZK_REQUIRE(M >= 0 && F >= 0 && K >= 0, ZK_EINVAL, "zk_gemm_swiglu: bad shape");
  ZK_REQUIRE(ld_x >= K && ld_w >= K && ld_gu >= F && ld_z >= F && (zt == nullptr || ld_zt >= M),
             ZK_EINVAL, "zk_gemm_swiglu: bad leading dimension");
  if (M == 0 || F == 0) return ZK_OK;
  ZK_REQUIRE(K > 0 && K % C::BK == 0, ZK_EUNSUPPORTED,
             "zk_gemm_swiglu: K must be a positive multiple of %d (got %lld)", C::BK,
             (long long)K);
  ZK_REQUIRE(M % 8 == 0 && F % 8 == 0, ZK_EUNSUPPORTED,
             "zk_gemm_swiglu: M and F must be multiples of 8 (got %lld, %lld)", (long long)M,
             (long long)F);
  const int64_t lds[] = {ld_x, ld_w, ld_gu, ld_z, zt ? ld_zt : 8};
  for (int64_t ld : lds)
    ZK_REQUIRE(ld % 8 == 0, ZK_EALIGN, "zk_gemm_swiglu: leading dimensions must be multiples of 8");
  const void* ptrs[] = {x, w_gate, w_up, g_out, u_out, z};
  for (const void* p : ptrs) {
    ZK_REQUIRE(p != nullptr, ZK_EINVAL, "zk_gemm_swiglu: null pointer");
    ZK_REQUIRE(aligned(p, 16), ZK_EALIGN, "zk_gemm_swiglu: operands must be 16-byte aligned");
  }
  ZK_REQUIRE(zt == nullptr || aligned(zt, 16), ZK_EALIGN,
             "zk_gemm_swiglu: operands must be 16-byte aligned");
  // the tile loaders keep a 32-row span of one operand in a 32-bit byte offset
  ZK_REQUIRE(ld_x < (int64_t(1) << 26) && ld_w < (int64_t(1) << 26), ZK_EUNSUPPORTED,
             "zk_gemm_swiglu: leading dimension out of range");
  if (zk_gemm_swiglu_tiled_supported(M, F, K) && ld_x < (int64_t(1) << 22) &&
      ld_w < (int64_t(1) << 22))
    return zk_gemm_swiglu_tiled(x, ld_x, w_gate, w_up, ld_w, g_out, u_out, ld_gu, z, ld_z, zt,
                                ld_zt, M, F, K, dtype, stream);
  const int64_t n_wg = ((M + C::BM - 1) / C::BM) * ((F + C::BF - 1) / C::BF);
  ZK_REQUIRE(n_wg < 0x7fffffffLL, ZK_EINVAL, "zk_gemm_swiglu: grid too large");
  hipStream_t s = as_stream(stream);
  if (dtype == ZK_BF16)
    hipLaunchKernelGGL(gemm_swiglu_kernel<bf16>, dim3(static_cast<unsigned>(n_wg)), dim3(256), 0,
                       s, (const bf16*)x, ld_x, (const bf16*)w_gate, (const bf16*)w_up, ld_w,
                       (bf16*)g_out, (bf16*)u_out, ld_gu, (bf16*)z, ld_z, (bf16*)zt, ld_zt, M, F,
                       K);
  else
    hipLaunchKernelGGL(gemm_swiglu_kernel<f16>, dim3(static_cast<unsigned>(n_wg)), dim3(256), 0,
                       s, (const f16*)x, ld_x, (const f16*)w_gate, (const f16*)w_up, ld_w,
                       (f16*)g_out, (f16*)u_out, ld_gu, (f16*)z, ld_z, (f16*)zt, ld_zt, M, F, K);
  return launch_status("zk_gemm_swiglu");
}
