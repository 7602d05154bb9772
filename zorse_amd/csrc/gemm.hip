// Projection GEMM entry points (zk_gemm, zk_gemm_nt, the SwiGLU-epilogue
// launch); the kernels and their design are in gemm_kernels.h.  The tiled
// forms with a K-major operand are launched from gemm_kmajor.hip.
#include <type_traits>

#include "gemm_kernels.h"

namespace zk {

// Whether the 256 x 256 pipeline takes a launch: 2-byte type, M and N
// multiples of 256, K a multiple of 128 and at least 256, leading dimensions
// multiples of 8 (16-byte tile rows and stores), and every tile of an operand
// within reach of one buffer resource: 256 rows of an NT operand or 64 rows
// of a K-major one below 2 GiB (lda, ldb below 2^22 / 2^24 elements).
// Pointer alignment is checked by the caller.
static bool tiled_takes(int64_t M, int64_t N, int64_t K, int64_t lda, int a_km, int64_t ldb,
                        int b_km, int64_t ldc, int64_t ldr, int dtype) {
  if (dtype != ZK_BF16 && dtype != ZK_F16) return false;
  if (!(M > 0 && N > 0 && M % gemm::BM == 0 && N % gemm::BN == 0 && K % (2 * gemm::BK) == 0 &&
        K >= 4 * gemm::BK))
    return false;
  if (lda % 8 || ldb % 8 || ldc % 8 || ldr % 8) return false;
  const int64_t lim_a = int64_t(1) << (a_km ? 24 : 22), lim_b = int64_t(1) << (b_km ? 24 : 22);
  return lda < lim_a && ldb < lim_b;
}

}  // namespace zk

using namespace zk;

extern "C" int zk_gemm_nt_supported(int64_t M, int64_t N, int64_t K) {
  return M > 0 && N > 0 && M % gemm::BM == 0 && N % gemm::BN == 0 && K % (2 * gemm::BK) == 0 &&
         K >= 4 * gemm::BK;
}

extern "C" int zk_gemm_path(int64_t M, int64_t N, int64_t K, int64_t lda, int a_kmajor,
                            int64_t ldb, int b_kmajor, int64_t ldc, int64_t ldr, int dtype) {
  ZK_REQUIRE(valid_dtype(dtype), ZK_EDTYPE, "zk_gemm_path: bad dtype %d", dtype);
  return tiled_takes(M, N, K, lda, a_kmajor != 0, ldb, b_kmajor != 0, ldc, ldr < 0 ? 8 : ldr,
                     dtype)
             ? ZK_GEMM_TILED
             : ZK_GEMM_GENERAL;
}

namespace {

template <typename T, bool AKM, bool BKM>
void launch_gemm(bool tiled, const gemm::GemmArgs& ga, hipStream_t s) {
  if constexpr (sizeof(T) == 2) {
    if (tiled) {
      if constexpr (AKM || BKM) {
        gemm::launch_tiled_kmajor(std::is_same<T, bf16>::value, AKM, BKM, ga, s);
      } else {
        const int64_t nwg = (ga.M / gemm::BM) * (ga.N / gemm::BN);
        if (gemm::half_tiles(nwg))
          hipLaunchKernelGGL((gemm::gemm_tiled_kernel<T, 0, false, false, 4>),
                             dim3(static_cast<unsigned>(2 * nwg)), dim3(256), 0, s, ga);
        else
          hipLaunchKernelGGL((gemm::gemm_tiled_kernel<T, 0, false, false>),
                             dim3(static_cast<unsigned>(nwg)), dim3(256), 0, s, ga);
      }
      return;
    }
  }
  {
    const int64_t nwg = ((ga.M + gemm::GBM - 1) / gemm::GBM) * ((ga.N + gemm::GBM - 1) / gemm::GBM);
    hipLaunchKernelGGL((gemm::gemm_gen_kernel<T, AKM, BKM>), dim3(static_cast<unsigned>(nwg)),
                       dim3(256), 0, s, ga);
  }
}

template <typename T>
void launch_layout(bool tiled, int a_km, int b_km, const gemm::GemmArgs& ga, hipStream_t s) {
  if (!a_km && !b_km)
    launch_gemm<T, false, false>(tiled, ga, s);
  else if (!a_km && b_km)
    launch_gemm<T, false, true>(tiled, ga, s);
  else if (a_km && b_km)
    launch_gemm<T, true, true>(tiled, ga, s);
  else
    launch_gemm<T, true, false>(tiled, ga, s);
}

}  // namespace

extern "C" int zk_gemm(const void* a, int64_t lda, int a_kmajor, const void* b, int64_t ldb,
                       int b_kmajor, void* c, int64_t ldc, const void* r, int64_t ldr, int64_t M,
                       int64_t N, int64_t K, int dtype, zk_stream_t stream) {
  ZK_REQUIRE(valid_dtype(dtype), ZK_EDTYPE, "zk_gemm: bad dtype %d", dtype);
  ZK_REQUIRE(M >= 0 && N >= 0 && K >= 0, ZK_EINVAL, "zk_gemm: bad shape");
  const int a_km = a_kmajor != 0, b_km = b_kmajor != 0;
  // an [M, K] operand needs ld >= K, a K-major [K, M] one ld >= M
  ZK_REQUIRE(lda >= (a_km ? M : K) && ldb >= (b_km ? N : K) && ldc >= N &&
                 (r == nullptr || ldr >= N),
             ZK_EINVAL, "zk_gemm: bad leading dimension");
  if (M == 0 || N == 0) return ZK_OK;
  ZK_REQUIRE(c != nullptr && (K == 0 || (a != nullptr && b != nullptr)), ZK_EINVAL,
             "zk_gemm: null pointer");
  const int eb = dtype_bytes(dtype);
  const void* ptrs[] = {a, b, c, r};
  for (const void* p : ptrs)
    ZK_REQUIRE(p == nullptr || aligned(p, eb), ZK_EALIGN,
               "zk_gemm: operands must be aligned to their element size");
  const int64_t rows_a = a_km ? K : M, rows_b = b_km ? K : N;
  // every index the kernels form stays below 2^62
  ZK_REQUIRE(lda < (int64_t(1) << 40) && ldb < (int64_t(1) << 40) && ldc < (int64_t(1) << 40) &&
                 (r == nullptr || ldr < (int64_t(1) << 40)) && rows_a < (int64_t(1) << 40) &&
                 rows_b < (int64_t(1) << 40) && M < (int64_t(1) << 40),
             ZK_EINVAL, "zk_gemm: sizes out of range");
  bool tiled = tiled_takes(M, N, K, lda, a_km, ldb, b_km, ldc, r ? ldr : 8, dtype);
  for (const void* p : ptrs) tiled = tiled && (p == nullptr || aligned(p, 16));
  const int64_t nwg = tiled ? (M / gemm::BM) * (N / gemm::BN)
                            : ((M + gemm::GBM - 1) / gemm::GBM) * ((N + gemm::GBM - 1) / gemm::GBM);
  ZK_REQUIRE(nwg < 0x7fffffffLL, ZK_EINVAL, "zk_gemm: grid too large");
  gemm::GemmArgs ga{};
  ga.a = a;
  ga.lda = lda;
  ga.b = b;
  ga.ldb = ldb;
  ga.c = c;
  ga.ldc = ldc;
  ga.r = r;
  ga.ldr = ldr;
  ga.M = M;
  ga.N = N;
  ga.K = K;
  hipStream_t s = as_stream(stream);
  if (dtype == ZK_BF16)
    launch_layout<bf16>(tiled, a_km, b_km, ga, s);
  else if (dtype == ZK_F16)
    launch_layout<f16>(tiled, a_km, b_km, ga, s);
  else
    launch_layout<float>(false, a_km, b_km, ga, s);
  return launch_status("zk_gemm");
}

extern "C" int zk_gemm_nt(const void* a, int64_t lda, const void* b, int64_t ldb, void* c,
                          int64_t ldc, const void* r, int64_t ldr, int64_t M, int64_t N,
                          int64_t K, int dtype, zk_stream_t stream) {
  return zk_gemm(a, lda, 0, b, ldb, 0, c, ldc, r, ldr, M, N, K, dtype, stream);
}

// The q|k|v projection with the rotary embedding applied in the GEMM's
// epilogue (EPI 2) when the 256 x 256 pipeline takes the launch; otherwise
// zk_gemm followed by zk_rope on the rotated columns, which rounds the same.
extern "C" int zk_gemm_rope(const void* a, int64_t lda, const void* b, int64_t ldb, void* c,
                            int64_t ldc, int64_t M, int64_t N, int64_t K, int64_t S,
                            int64_t rot_cols, int64_t head_dim, const float* cos,
                            const float* sin, int64_t n_pos, const int64_t* positions,
                            int pairing, int dtype, zk_stream_t stream) {
  ZK_REQUIRE(valid_dtype(dtype), ZK_EDTYPE, "zk_gemm_rope: bad dtype %d", dtype);
  ZK_REQUIRE(pairing == ZK_ROPE_HALF || pairing == ZK_ROPE_INTERLEAVED, ZK_EINVAL,
             "zk_gemm_rope: bad pairing %d", pairing);
  ZK_REQUIRE(M >= 0 && N >= 0 && K >= 0 && S > 0 && M % S == 0, ZK_EINVAL,
             "zk_gemm_rope: bad shape (M = %lld rows must be whole sequences of S = %lld)",
             (long long)M, (long long)S);
  ZK_REQUIRE(head_dim > 0 && head_dim % 2 == 0 && rot_cols >= 0 && rot_cols % head_dim == 0 &&
                 rot_cols <= N,
             ZK_EINVAL, "zk_gemm_rope: rotated columns %lld must be whole heads of %lld within N",
             (long long)rot_cols, (long long)head_dim);
  ZK_REQUIRE(cos != nullptr && sin != nullptr && n_pos > 0, ZK_EINVAL,
             "zk_gemm_rope: null or empty rotation table");
  ZK_REQUIRE(positions != nullptr || n_pos >= S, ZK_EINVAL,
             "zk_gemm_rope: table has %lld positions < S = %lld", (long long)n_pos, (long long)S);
  ZK_REQUIRE(lda >= K && ldb >= K && ldc >= N, ZK_EINVAL, "zk_gemm_rope: bad leading dimension");
  ZK_REQUIRE(lda < (int64_t(1) << 40) && ldb < (int64_t(1) << 40) && ldc < (int64_t(1) << 40) &&
                 M < (int64_t(1) << 40) && N < (int64_t(1) << 40),
             ZK_EINVAL, "zk_gemm_rope: sizes out of range");
  if (M == 0 || N == 0) return ZK_OK;
  ZK_REQUIRE(c != nullptr && (K == 0 || (a != nullptr && b != nullptr)), ZK_EINVAL,
             "zk_gemm_rope: null pointer");
  const bool epi = tiled_takes(M, N, K, lda, 0, ldb, 0, ldc, 8, dtype) && aligned(a, 16) &&
                   aligned(b, 16) && aligned(c, 16) && (head_dim == 64 || head_dim == 128) &&
                   rot_cols % 128 == 0 && aligned(cos, 16) && aligned(sin, 16) &&
                   S >= 128 && S < (int64_t(1) << 30) && n_pos < (int64_t(1) << 24) &&
                   (M / gemm::BM) * (N / gemm::BN) < 0x7fffffffLL;
  if (!epi) {
    const int rc = zk_gemm(a, lda, 0, b, ldb, 0, c, ldc, nullptr, 0, M, N, K, dtype, stream);
    if (rc != ZK_OK || rot_cols == 0) return rc;
    // the rotated heads as the "q" heads of a [B, S, H, d] view of c
    return zk_rope(c, S * ldc, ldc, head_dim, nullptr, 0, 0, 0, M / S, S, rot_cols / head_dim,
                   0, head_dim, cos, sin, n_pos, positions, pairing, 0, dtype, stream);
  }
  gemm::GemmArgs ga{};
  ga.a = a;
  ga.lda = lda;
  ga.b = b;
  ga.ldb = ldb;
  ga.c = c;
  ga.ldc = ldc;
  ga.M = M;
  ga.N = N;
  ga.K = K;
  ga.rcos = cos;
  ga.rsin = sin;
  ga.rpos = positions;
  ga.rnpos = n_pos;
  ga.rS = S;
  ga.rcols = rot_cols;
  ga.rhalf = static_cast<int>(head_dim / 2);
  ga.rpair = pairing;
  const dim3 grid(static_cast<unsigned>((M / gemm::BM) * (N / gemm::BN)));
  hipStream_t s = as_stream(stream);
  if (dtype == ZK_BF16)
    hipLaunchKernelGGL((gemm::gemm_tiled_kernel<bf16, 2, false, false>), grid, dim3(256), 0, s, ga);
  else
    hipLaunchKernelGGL((gemm::gemm_tiled_kernel<f16, 2, false, false>), grid, dim3(256), 0, s, ga);
  return launch_status("zk_gemm_rope");
}

namespace zk {

// The gate|up projection with the SwiGLU epilogue on the 256 x 256 pipeline
// (zk_gemm_swiglu routes the shapes it takes here: M a multiple of 256, F of
// 128, K of 128 and at least 256, ld_x and ld_w below 2^22).  Arguments as
// zk_gemm_swiglu, already validated.
int zk_gemm_swiglu_tiled_supported(int64_t M, int64_t F, int64_t K) {
  return zk_gemm_nt_supported(M, 2 * F, K);
}

int zk_gemm_swiglu_tiled(const void* x, int64_t ld_x, const void* w_gate, const void* w_up,
                         int64_t ld_w, void* g_out, void* u_out, int64_t ld_gu, void* z,
                         int64_t ld_z, void* zt, int64_t ld_zt, int64_t M, int64_t F, int64_t K,
                         int dtype, zk_stream_t stream) {
  gemm::GemmArgs ga{};
  ga.a = x;
  ga.lda = ld_x;
  ga.b = w_gate;
  ga.b2 = w_up;
  ga.ldb = ld_w;
  ga.c = g_out;
  ga.c2 = u_out;
  ga.ldc = ld_gu;
  ga.z = z;
  ga.ldz = ld_z;
  ga.zt = zt;
  ga.ldzt = ld_zt;
  ga.M = M;
  ga.N = 2 * F;
  ga.K = K;
  const int64_t nwg = (M / gemm::BM) * (2 * F / gemm::BN);
  hipStream_t s = as_stream(stream);
  if (dtype == ZK_BF16)
    hipLaunchKernelGGL((gemm::gemm_tiled_kernel<bf16, 1, false, false>),
                       dim3(static_cast<unsigned>(nwg)), dim3(256), 0, s, ga);
  else
    hipLaunchKernelGGL((gemm::gemm_tiled_kernel<f16, 1, false, false>),
                       dim3(static_cast<unsigned>(nwg)), dim3(256), 0, s, ga);
  return launch_status("zk_gemm_swiglu");
}

}  // namespace zk
