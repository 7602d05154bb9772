// SwiGLU activation (forward / backward) and dtype casts.
//
// Both are HBM-bound streams: 8 elements per thread per iteration (16-byte
// accesses for 2-byte types), grid-stride over rows x 8-column chunks.  The
// rounding points follow the reference's bf16/fp16 op sequence, silu(g)
// rounded to the storage type before the product, so that the fused kernel
// reproduces what torch computes op by op.
#include <initializer_list>

#include "vec.h"

namespace zk {

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

template <typename T>
__global__ __launch_bounds__(256) void swiglu_fwd_vec(
    const T* __restrict__ gate, const T* __restrict__ up, int64_t ld_in,
    T* __restrict__ z, int64_t ld_z, int64_t rows, int64_t cols) {
  // one workgroup per row (grid-stride over rows), 8 columns per thread-step
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x)
  for (int64_t c = threadIdx.x * 8; c < cols; c += 256 * 8) {
    float g[8], u[8], o[8];
    Vec8<T>::load(gate + r * ld_in + c, g);
    Vec8<T>::load(up + r * ld_in + c, u);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = round_to<T>(silu_f(g[i])) * u[i];
    Vec8<T>::store(z + r * ld_z + c, o);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_bwd_vec(
    const T* __restrict__ dz, int64_t ld_dz, const T* __restrict__ gate,
    const T* __restrict__ up, int64_t ld_in, T* __restrict__ dgate,
    T* __restrict__ dup, int64_t ld_out, int64_t rows, int64_t cols) {
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x)
  for (int64_t c = threadIdx.x * 8; c < cols; c += 256 * 8) {
    float d[8], g[8], u[8], dg[8], du[8];
    Vec8<T>::load(dz + r * ld_dz + c, d);
    Vec8<T>::load(gate + r * ld_in + c, g);
    Vec8<T>::load(up + r * ld_in + c, u);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float den = 1.0f + expf(-g[i]);
      const float sg = 1.0f / den;
      const float s = round_to<T>(g[i] / den);
      du[i] = d[i] * s;
      const float ds = round_to<T>(d[i] * u[i]);
      dg[i] = ds * sg * (1.0f + g[i] * (1.0f - sg));
    }
    Vec8<T>::store(dgate + r * ld_out + c, dg);
    Vec8<T>::store(dup + r * ld_out + c, du);
  }
}

// SwiGLU with a transposed copy of its output (2-byte types).  The weight
// gradient of the projection that consumes the output reduces over tokens, and
// the GEMM is fastest with both operands token-contiguous, so the producer
// writes out^T [cols, rows] next to out [rows, cols]: the transposed copy costs
// one extra write instead of a separate read + write pass.
//
// A workgroup owns a 64-token x 64-column tile: 16-byte loads (8 columns per
// thread, 2 chunks per thread), the row-major result stored directly, then
// the tile is staged in LDS (row pitch 66 elements, so that the column reads
// of the transpose spread over the banks) and written back as 64
// rows of 64 tokens with 16-byte stores.  Requires rows % 8 == 0 and
// cols % 8 == 0; partial tiles at the edges are masked per 8-element chunk.
template <typename T>
struct TTile {
  static constexpr int R = 64, C = 64, P = C + 2;  // tile rows (tokens), cols, LDS pitch
};

// Writes the LDS tile (row-major, pitch P, R x C) transposed: out^T[c][r0 + r].
template <typename T>
__device__ __forceinline__ void store_tile_t(const T (*tile)[TTile<T>::P], T* __restrict__ out_t,
                                             int64_t ld_t, int64_t r0, int64_t c0, int64_t rows,
                                             int64_t cols) {
  constexpr int R = TTile<T>::R;
  // thread -> (column cc, 8-token chunk rr): 64 columns x 8 chunks = 512 items
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int item = it * 256 + threadIdx.x;
    const int cc = item / (R / 8), rr = (item % (R / 8)) * 8;
    if (c0 + cc < cols && r0 + rr < rows) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = to_f32(tile[rr + e][cc]);
      Vec8<T>::store(out_t + (c0 + cc) * ld_t + r0 + rr, v);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_fwd_t(
    const T* __restrict__ gate, const T* __restrict__ up, int64_t ld_in, T* __restrict__ z,
    int64_t ld_z, T* __restrict__ zt, int64_t ld_zt, int64_t rows, int64_t cols) {
  typedef TTile<T> TT;
  __shared__ T tile[TT::R][TT::P];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * TT::R;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * TT::C;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int item = it * 256 + threadIdx.x;          // 64 rows x 8 chunks
    const int rr = item / (TT::C / 8), cc = (item % (TT::C / 8)) * 8;
    const int64_t r = r0 + rr, c = c0 + cc;
    if (r < rows && c < cols) {
      float g[8], u[8], o[8];
      Vec8<T>::load(gate + r * ld_in + c, g);
      Vec8<T>::load(up + r * ld_in + c, u);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = round_to<T>(silu_f(g[i])) * u[i];
      Vec8<T>::store(z + r * ld_z + c, o);
#pragma unroll
      for (int i = 0; i < 8; ++i) tile[rr][cc + i] = static_cast<T>(o[i]);
    }
  }
  __syncthreads();
  store_tile_t<T>(tile, zt, ld_zt, r0, c0, rows, cols);
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_bwd_t(
    const T* __restrict__ dz, int64_t ld_dz, const T* __restrict__ gate,
    const T* __restrict__ up, int64_t ld_in, T* __restrict__ dgate, T* __restrict__ dup,
    int64_t ld_out, T* __restrict__ dgate_t, T* __restrict__ dup_t, int64_t ld_t, int64_t rows,
    int64_t cols) {
  typedef TTile<T> TT;
  __shared__ T tg[TT::R][TT::P];
  __shared__ T tu[TT::R][TT::P];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * TT::R;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * TT::C;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int item = it * 256 + threadIdx.x;
    const int rr = item / (TT::C / 8), cc = (item % (TT::C / 8)) * 8;
    const int64_t r = r0 + rr, c = c0 + cc;
    if (r < rows && c < cols) {
      float d[8], g[8], u[8], dg[8], du[8];
      Vec8<T>::load(dz + r * ld_dz + c, d);
      Vec8<T>::load(gate + r * ld_in + c, g);
      Vec8<T>::load(up + r * ld_in + c, u);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float den = 1.0f + expf(-g[i]);
        const float sg = 1.0f / den;
        const float sv = round_to<T>(g[i] / den);
        du[i] = d[i] * sv;
        const float ds = round_to<T>(d[i] * u[i]);
        dg[i] = ds * sg * (1.0f + g[i] * (1.0f - sg));
      }
      Vec8<T>::store(dgate + r * ld_out + c, dg);
      Vec8<T>::store(dup + r * ld_out + c, du);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        tg[rr][cc + i] = static_cast<T>(dg[i]);
        tu[rr][cc + i] = static_cast<T>(du[i]);
      }
    }
  }
  __syncthreads();
  store_tile_t<T>(tg, dgate_t, ld_t, r0, c0, rows, cols);
  store_tile_t<T>(tu, dup_t, ld_t, r0, c0, rows, cols);
}

// Scalar fallbacks (any width / alignment).
__global__ __launch_bounds__(256) void swiglu_fwd_scalar(
    const void* __restrict__ gate, const void* __restrict__ up, int64_t ld_in,
    void* __restrict__ z, int64_t ld_z, int64_t rows, int64_t cols, int dt) {
  const int64_t total = rows * cols;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       t < total; t += stride) {
    const int64_t r = t / cols, c = t - r * cols;
    const float g = load_dt(gate, r * ld_in + c, dt);
    const float u = load_dt(up, r * ld_in + c, dt);
    float s = silu_f(g);
    if (dt == ZK_BF16) s = round_to<bf16>(s);
    else if (dt == ZK_F16) s = round_to<f16>(s);
    store_dt(z, r * ld_z + c, dt, s * u);
  }
}

__global__ __launch_bounds__(256) void swiglu_bwd_scalar(
    const void* __restrict__ dz, int64_t ld_dz, const void* __restrict__ gate,
    const void* __restrict__ up, int64_t ld_in, void* __restrict__ dgate,
    void* __restrict__ dup, int64_t ld_out, int64_t rows, int64_t cols,
    int dt) {
  const int64_t total = rows * cols;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       t < total; t += stride) {
    const int64_t r = t / cols, c = t - r * cols;
    const float d = load_dt(dz, r * ld_dz + c, dt);
    const float g = load_dt(gate, r * ld_in + c, dt);
    const float u = load_dt(up, r * ld_in + c, dt);
    const float den = 1.0f + expf(-g);
    const float sg = 1.0f / den;
    float s = g / den, ds = d * u;
    if (dt == ZK_BF16) { s = round_to<bf16>(s); ds = round_to<bf16>(ds); }
    else if (dt == ZK_F16) { s = round_to<f16>(s); ds = round_to<f16>(ds); }
    store_dt(dup, r * ld_out + c, dt, d * s);
    store_dt(dgate, r * ld_out + c, dt, ds * sg * (1.0f + g * (1.0f - sg)));
  }
}

// y = round(x) or y = round(y + x)
template <typename TX, typename TY>
__global__ __launch_bounds__(256) void cast_vec(const TX* __restrict__ x,
                                                TY* __restrict__ y, int64_t n8,
                                                int accumulate) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       t < n8; t += stride) {
    float v[8];
    Vec8<TX>::load(x + t * 8, v);
    if (accumulate) {
      float w[8];
      Vec8<TY>::load(y + t * 8, w);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] += w[i];
    }
    Vec8<TY>::store(y + t * 8, v);
  }
}

__global__ __launch_bounds__(256) void cast_scalar(const void* __restrict__ x,
                                                   int xdt, void* __restrict__ y,
                                                   int ydt, int64_t begin,
                                                   int64_t n, int accumulate) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = begin + static_cast<int64_t>(blockIdx.x) * blockDim.x +
                   threadIdx.x;
       i < n; i += stride) {
    float v = load_dt(x, i, xdt);
    if (accumulate) v += load_dt(y, i, ydt);
    store_dt(y, i, ydt, v);
  }
}

static int grid_for(int64_t work) {
  const int64_t cap = static_cast<int64_t>(device_cus()) * 16;
  int64_t g = (work + 255) / 256;
  if (g > cap) g = cap;
  return static_cast<int>(g < 1 ? 1 : g);
}

template <typename TX>
static void cast_dispatch_y(const void* x, void* y, int ydt, int64_t n8, int acc,
                            int grid, hipStream_t s) {
  if (ydt == ZK_F32)
    hipLaunchKernelGGL((cast_vec<TX, float>), dim3(grid), dim3(256), 0, s, (const TX*)x, (float*)y, n8, acc);
  else if (ydt == ZK_BF16)
    hipLaunchKernelGGL((cast_vec<TX, bf16>), dim3(grid), dim3(256), 0, s, (const TX*)x, (bf16*)y, n8, acc);
  else
    hipLaunchKernelGGL((cast_vec<TX, f16>), dim3(grid), dim3(256), 0, s, (const TX*)x, (f16*)y, n8, acc);
}

}  // namespace zk

using namespace zk;

extern "C" int zk_swiglu_fwd(const void* gate, const void* up, int64_t ld_in,
                             void* z, int64_t ld_z, int64_t rows, int64_t cols,
                             int dtype, zk_stream_t stream) {
  ZK_REQUIRE(valid_dtype(dtype), ZK_EDTYPE, "zk_swiglu_fwd: bad dtype %d", dtype);
  ZK_REQUIRE(rows >= 0 && cols >= 0 && ld_in >= cols && ld_z >= cols, ZK_EINVAL,
             "zk_swiglu_fwd: bad shape rows=%lld cols=%lld ld_in=%lld ld_z=%lld",
             (long long)rows, (long long)cols, (long long)ld_in, (long long)ld_z);
  if (rows == 0 || cols == 0) return ZK_OK;
  ZK_REQUIRE(gate && up && z, ZK_EINVAL, "zk_swiglu_fwd: null pointer");
  hipStream_t s = as_stream(stream);
  const bool vec = cols % 8 == 0 && ld_in % 8 == 0 && ld_z % 8 == 0 &&
                   aligned(gate, 16) && aligned(up, 16) && aligned(z, 16);
  if (vec) {
    const int grid = static_cast<int>(rows < 0x7fffffff ? rows : 0x7fffffff);  // a row per workgroup
    if (dtype == ZK_BF16)
      hipLaunchKernelGGL(swiglu_fwd_vec<bf16>, dim3(grid), dim3(256), 0, s, (const bf16*)gate, (const bf16*)up, ld_in, (bf16*)z, ld_z, rows, cols);
    else if (dtype == ZK_F16)
      hipLaunchKernelGGL(swiglu_fwd_vec<f16>, dim3(grid), dim3(256), 0, s, (const f16*)gate, (const f16*)up, ld_in, (f16*)z, ld_z, rows, cols);
    else
      hipLaunchKernelGGL(swiglu_fwd_vec<float>, dim3(grid), dim3(256), 0, s, (const float*)gate, (const float*)up, ld_in, (float*)z, ld_z, rows, cols);
  } else {
    hipLaunchKernelGGL(swiglu_fwd_scalar, dim3(grid_for(rows * cols)), dim3(256), 0, s, gate, up, ld_in, z, ld_z, rows, cols, dtype);
  }
  return launch_status("zk_swiglu_fwd");
}

extern "C" int zk_swiglu_bwd(const void* dz, int64_t ld_dz, const void* gate,
                             const void* up, int64_t ld_in, void* dgate,
                             void* dup, int64_t ld_out, int64_t rows,
                             int64_t cols, int dtype, zk_stream_t stream) {
  ZK_REQUIRE(valid_dtype(dtype), ZK_EDTYPE, "zk_swiglu_bwd: bad dtype %d", dtype);
  ZK_REQUIRE(rows >= 0 && cols >= 0 && ld_in >= cols && ld_dz >= cols &&
                 ld_out >= cols,
             ZK_EINVAL, "zk_swiglu_bwd: bad shape");
  if (rows == 0 || cols == 0) return ZK_OK;
  ZK_REQUIRE(dz && gate && up && dgate && dup, ZK_EINVAL, "zk_swiglu_bwd: null pointer");
  hipStream_t s = as_stream(stream);
  const bool vec = cols % 8 == 0 && ld_in % 8 == 0 && ld_dz % 8 == 0 &&
                   ld_out % 8 == 0 && aligned(dz, 16) && aligned(gate, 16) &&
                   aligned(up, 16) && aligned(dgate, 16) && aligned(dup, 16);
  if (vec) {
    const int grid = static_cast<int>(rows < 0x7fffffff ? rows : 0x7fffffff);  // a row per workgroup
    if (dtype == ZK_BF16)
      hipLaunchKernelGGL(swiglu_bwd_vec<bf16>, dim3(grid), dim3(256), 0, s, (const bf16*)dz, ld_dz, (const bf16*)gate, (const bf16*)up, ld_in, (bf16*)dgate, (bf16*)dup, ld_out, rows, cols);
    else if (dtype == ZK_F16)
      hipLaunchKernelGGL(swiglu_bwd_vec<f16>, dim3(grid), dim3(256), 0, s, (const f16*)dz, ld_dz, (const f16*)gate, (const f16*)up, ld_in, (f16*)dgate, (f16*)dup, ld_out, rows, cols);
    else
      hipLaunchKernelGGL(swiglu_bwd_vec<float>, dim3(grid), dim3(256), 0, s, (const float*)dz, ld_dz, (const float*)gate, (const float*)up, ld_in, (float*)dgate, (float*)dup, ld_out, rows, cols);
  } else {
    hipLaunchKernelGGL(swiglu_bwd_scalar, dim3(grid_for(rows * cols)), dim3(256), 0, s, dz, ld_dz, gate, up, ld_in, dgate, dup, ld_out, rows, cols, dtype);
  }
  return launch_status("zk_swiglu_bwd");
}

// Shared checks of the transposed-output variants: 2-byte type, 16-byte
// aligned operands, rows / cols / leading dimensions multiples of 8, grid in range.
static int check_t_args(const char* who, int dtype, int64_t rows, int64_t cols,
                        std::initializer_list<int64_t> lds,
                        std::initializer_list<const void*> ptrs) {
  ZK_REQUIRE(dtype == ZK_BF16 || dtype == ZK_F16, ZK_EDTYPE,
             "%s: 2-byte dtypes only (got %d)", who, dtype);
  ZK_REQUIRE(rows >= 0 && cols >= 0, ZK_EINVAL, "%s: bad shape", who);
  ZK_REQUIRE(rows % 8 == 0 && cols % 8 == 0, ZK_EUNSUPPORTED,
             "%s: rows and cols must be multiples of 8 (got %lld, %lld)", who,
             (long long)rows, (long long)cols);
  for (int64_t ld : lds)
    ZK_REQUIRE(ld % 8 == 0, ZK_EALIGN, "%s: leading dimensions must be multiples of 8", who);
  for (const void* p : ptrs) {
    ZK_REQUIRE(p != nullptr, ZK_EINVAL, "%s: null pointer", who);
    ZK_REQUIRE(aligned(p, 16), ZK_EALIGN, "%s: operands must be 16-byte aligned", who);
  }
  ZK_REQUIRE((rows + 63) / 64 < 65536 && (cols + 63) / 64 < 0x7fffffffLL, ZK_EINVAL,
             "%s: grid too large", who);
  return ZK_OK;
}

extern "C" int zk_swiglu_fwd_t(const void* gate, const void* up, int64_t ld_in, void* z,
                               int64_t ld_z, void* zt, int64_t ld_zt, int64_t rows,
                               int64_t cols, int dtype, zk_stream_t stream) {
  ZK_REQUIRE(ld_in >= cols && ld_z >= cols && ld_zt >= rows, ZK_EINVAL,
             "zk_swiglu_fwd_t: bad leading dimension");
  if (rows == 0 || cols == 0) return ZK_OK;
  int rc = check_t_args("zk_swiglu_fwd_t", dtype, rows, cols, {ld_in, ld_z, ld_zt},
                        {gate, up, z, zt});
  if (rc != ZK_OK) return rc;
  hipStream_t s = as_stream(stream);
  const dim3 grid(static_cast<unsigned>((cols + 63) / 64), static_cast<unsigned>((rows + 63) / 64));
  if (dtype == ZK_BF16)
    hipLaunchKernelGGL(swiglu_fwd_t<bf16>, grid, dim3(256), 0, s, (const bf16*)gate,
                       (const bf16*)up, ld_in, (bf16*)z, ld_z, (bf16*)zt, ld_zt, rows, cols);
  else
    hipLaunchKernelGGL(swiglu_fwd_t<f16>, grid, dim3(256), 0, s, (const f16*)gate,
                       (const f16*)up, ld_in, (f16*)z, ld_z, (f16*)zt, ld_zt, rows, cols);
  return launch_status("zk_swiglu_fwd_t");
}

extern "C" int zk_swiglu_bwd_t(const void* dz, int64_t ld_dz, const void* gate,
                               const void* up, int64_t ld_in, void* dgate, void* dup,
                               int64_t ld_out, void* dgate_t, void* dup_t, int64_t ld_t,
                               int64_t rows, int64_t cols, int dtype, zk_stream_t stream) {
  ZK_REQUIRE(ld_in >= cols && ld_dz >= cols && ld_out >= cols && ld_t >= rows, ZK_EINVAL,
             "zk_swiglu_bwd_t: bad leading dimension");
  if (rows == 0 || cols == 0) return ZK_OK;
  int rc = check_t_args("zk_swiglu_bwd_t", dtype, rows, cols, {ld_dz, ld_in, ld_out, ld_t},
                        {dz, gate, up, dgate, dup, dgate_t, dup_t});
  if (rc != ZK_OK) return rc;
  hipStream_t s = as_stream(stream);
  const dim3 grid(static_cast<unsigned>((cols + 63) / 64), static_cast<unsigned>((rows + 63) / 64));
  if (dtype == ZK_BF16)
    hipLaunchKernelGGL(swiglu_bwd_t<bf16>, grid, dim3(256), 0, s, (const bf16*)dz, ld_dz,
                       (const bf16*)gate, (const bf16*)up, ld_in, (bf16*)dgate, (bf16*)dup,
                       ld_out, (bf16*)dgate_t, (bf16*)dup_t, ld_t, rows, cols);
  else
    hipLaunchKernelGGL(swiglu_bwd_t<f16>, grid, dim3(256), 0, s, (const f16*)dz, ld_dz,
                       (const f16*)gate, (const f16*)up, ld_in, (f16*)dgate, (f16*)dup,
                       ld_out, (f16*)dgate_t, (f16*)dup_t, ld_t, rows, cols);
  return launch_status("zk_swiglu_bwd_t");
}

extern "C" int zk_cast(const void* x, int x_dtype, void* y, int y_dtype,
                       int64_t n, int accumulate, zk_stream_t stream) {
  ZK_REQUIRE(valid_dtype(x_dtype) && valid_dtype(y_dtype), ZK_EDTYPE,
             "zk_cast: bad dtype (%d, %d)", x_dtype, y_dtype);
  ZK_REQUIRE(n >= 0, ZK_EINVAL, "zk_cast: negative n");
  if (n == 0) return ZK_OK;
  ZK_REQUIRE(x && y, ZK_EINVAL, "zk_cast: null pointer");
  hipStream_t s = as_stream(stream);
  const bool vec = aligned(x, 8 * dtype_bytes(x_dtype)) &&
                   aligned(y, 8 * dtype_bytes(y_dtype));
  const int64_t n8 = vec ? n / 8 : 0;
  if (n8 > 0) {
    const int grid = grid_for(n8);
    if (x_dtype == ZK_F32) cast_dispatch_y<float>(x, y, y_dtype, n8, accumulate, grid, s);
    else if (x_dtype == ZK_BF16) cast_dispatch_y<bf16>(x, y, y_dtype, n8, accumulate, grid, s);
    else cast_dispatch_y<f16>(x, y, y_dtype, n8, accumulate, grid, s);
  }
  if (n8 * 8 < n)
    hipLaunchKernelGGL(cast_scalar, dim3(grid_for(n - n8 * 8)), dim3(256), 0, s,
                       x, x_dtype, y, y_dtype, n8 * 8, n, accumulate);
  return launch_status("zk_cast");
}
