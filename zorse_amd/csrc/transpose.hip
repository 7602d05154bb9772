// Out-of-place 2-D transpose, dst[c][r] = src[r][c].
//
// Used on the backward's projection gradients: the weight gradient
// dW = dY^T X reduces over the token dimension, which is the strided one of
// both row-major operands; with dY^T materialised the GEMM runs in the
// layout whose operands stream along the reduction (the one the other
// projection GEMMs use), which more than pays for this pass.
//
// A workgroup moves one TR x TC tile through LDS: 16-byte row loads, a
// padded LDS tile (row pitch TC + 2 elements, so the column reads of a wave
// spread over the banks), and 16-byte stores of 8 consecutive source rows.
// Two shapes: 128 x 128 tiles from 512 threads (256-byte row segments each
// way and 32 KB in flight per workgroup) when the source has at least as many
// rows as columns -- the activations' [T, h] and the taller weights -- and
// 64 x 64 tiles from 256 threads otherwise, where the large tile measured
// slower (4096 x 4096: 16.2 -> 13.8 us; 22016 x 4096: 75.8 -> 74.1 us;
// 4096 x 11008: 37.4 -> 39.8 us).
#include "zk_common.h"

namespace zk {

template <typename T>
struct Pack8;  // 8 elements of a 2-byte type as one 16-byte word
template <>
struct Pack8<bf16> { typedef bf16x8 type; };
template <>
struct Pack8<f16> { typedef f16x8 type; };

static constexpr int kTile = 64;  // tile of the element-wise kernel

template <typename T, int TR, int TC, int NT>
__global__ __launch_bounds__(NT) void transpose2_kernel(const T* __restrict__ src, int64_t ld_src,
                                                        T* __restrict__ dst, int64_t ld_dst,
                                                        int64_t rows, int64_t cols) {
  typedef typename Pack8<T>::type P8;
  constexpr int P = TC + 2;      // LDS row pitch
  constexpr int CR = TC / 8;     // 16-byte chunks per source row of the tile
  constexpr int CW = TR / 8;     // 16-byte chunks per destination row
  static_assert((TR * CR) % NT == 0 && (TC * CW) % NT == 0, "tile / thread mismatch");
  __shared__ T tile[TR * P];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * TR;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * TC;
  const int tid = threadIdx.x;
  const bool full = r0 + TR <= rows && c0 + TC <= cols;
  // load: TR rows x CR chunks of 8 elements
#pragma unroll
  for (int i = 0; i < TR * CR / NT; ++i) {
    const int q = tid + NT * i;
    const int r = q / CR, ch = q % CR;
    T v[8];
    if (full) {
      const P8 w = *reinterpret_cast<const P8*>(src + (r0 + r) * ld_src + c0 + 8 * ch);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = w[e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t gr = r0 + r, gc = c0 + 8 * ch + e;
        v[e] = gr < rows && gc < cols ? src[gr * ld_src + gc] : T(0.f);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[r * P + 8 * ch + e] = v[e];
  }
  __syncthreads();
  // store: TC destination rows (source columns) x CW chunks of 8 source rows
#pragma unroll
  for (int i = 0; i < TC * CW / NT; ++i) {
    const int q = tid + NT * i;
    const int c = q / CW, ch = q % CW;
    P8 w;
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = tile[(8 * ch + e) * P + c];
    if (full) {
      *reinterpret_cast<P8*>(dst + (c0 + c) * ld_dst + r0 + 8 * ch) = w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t gc = c0 + c, gr = r0 + 8 * ch + e;
        if (gc < cols && gr < rows) dst[gc * ld_dst + gr] = w[e];
      }
    }
  }
}

template <typename T, int TR, int TC, int NT>
static void launch_transpose2(const T* src, int64_t ld_src, T* dst, int64_t ld_dst, int64_t rows,
                              int64_t cols, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((cols + TC - 1) / TC),
                  static_cast<unsigned>((rows + TR - 1) / TR));
  hipLaunchKernelGGL((transpose2_kernel<T, TR, TC, NT>), grid, dim3(NT), 0, s, src, ld_src, dst,
                     ld_dst, rows, cols);
}

template <typename T>
static void transpose2(const void* src, int64_t ld_src, void* dst, int64_t ld_dst, int64_t rows,
                       int64_t cols, hipStream_t s) {
  if (rows >= cols)
    launch_transpose2<T, 128, 128, 512>(static_cast<const T*>(src), ld_src, static_cast<T*>(dst),
                                        ld_dst, rows, cols, s);
  else
    launch_transpose2<T, 64, 64, 256>(static_cast<const T*>(src), ld_src, static_cast<T*>(dst),
                                      ld_dst, rows, cols, s);
}

// fp32 (and any unaligned case of the 2-byte types goes through here too):
// the same tile with element accesses.
template <typename T>
__global__ __launch_bounds__(256) void transpose_scalar_kernel(const T* __restrict__ src,
                                                               int64_t ld_src, T* __restrict__ dst,
                                                               int64_t ld_dst, int64_t rows,
                                                               int64_t cols) {
  __shared__ T tile[kTile * (kTile + 1)];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * kTile;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kTile;
  for (int q = threadIdx.x; q < kTile * kTile; q += 256) {
    const int r = q / kTile, c = q % kTile;
    const int64_t gr = r0 + r, gc = c0 + c;
    tile[r * (kTile + 1) + c] = gr < rows && gc < cols ? src[gr * ld_src + gc] : T(0.f);
  }
  __syncthreads();
  for (int q = threadIdx.x; q < kTile * kTile; q += 256) {
    const int c = q / kTile, r = q % kTile;
    const int64_t gr = r0 + r, gc = c0 + c;
    if (gr < rows && gc < cols) dst[gc * ld_dst + gr] = tile[r * (kTile + 1) + c];
  }
}

}  // namespace zk

using namespace zk;

extern "C" int zk_transpose(const void* src, int64_t ld_src, void* dst, int64_t ld_dst,
                            int64_t rows, int64_t cols, int dtype, zk_stream_t stream) {
  ZK_REQUIRE(valid_dtype(dtype), ZK_EDTYPE, "zk_transpose: bad dtype %d", dtype);
  ZK_REQUIRE(rows >= 0 && cols >= 0 && ld_src >= cols && ld_dst >= rows, ZK_EINVAL,
             "zk_transpose: bad shape rows=%lld cols=%lld ld_src=%lld ld_dst=%lld",
             (long long)rows, (long long)cols, (long long)ld_src, (long long)ld_dst);
  if (rows == 0 || cols == 0) return ZK_OK;
  ZK_REQUIRE(src && dst, ZK_EINVAL, "zk_transpose: null pointer");
  ZK_REQUIRE(src != dst, ZK_EINVAL, "zk_transpose: in-place transpose is not supported");
  const int64_t gx = (cols + kTile - 1) / kTile, gy = (rows + kTile - 1) / kTile;
  ZK_REQUIRE(gx < 0x7fffffffLL && gy <= 65535, ZK_EINVAL, "zk_transpose: grid too large");
  hipStream_t s = as_stream(stream);
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  const bool vec = dtype != ZK_F32 && aligned(src, 16) && aligned(dst, 16) && ld_src % 8 == 0 &&
                   ld_dst % 8 == 0;
  if (vec && dtype == ZK_BF16)
    transpose2<bf16>(src, ld_src, dst, ld_dst, rows, cols, s);
  else if (vec)
    transpose2<f16>(src, ld_src, dst, ld_dst, rows, cols, s);
  else if (dtype == ZK_BF16)
    hipLaunchKernelGGL(transpose_scalar_kernel<bf16>, grid, dim3(256), 0, s, (const bf16*)src,
                       ld_src, (bf16*)dst, ld_dst, rows, cols);
  else if (dtype == ZK_F16)
    hipLaunchKernelGGL(transpose_scalar_kernel<f16>, grid, dim3(256), 0, s, (const f16*)src,
                       ld_src, (f16*)dst, ld_dst, rows, cols);
  else
    hipLaunchKernelGGL(transpose_scalar_kernel<float>, grid, dim3(256), 0, s, (const float*)src,
                       ld_src, (float*)dst, ld_dst, rows, cols);
  return launch_status("zk_transpose");
}
