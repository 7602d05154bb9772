// Cross-entropy over a vocabulary processed in column chunks, so the
// [tokens, vocab] logits never exist at once (the last pipeline stage's
// output layer + loss).
//
// zk_ce_fwd_chunk: for each row of a [rows, cols] chunk of logits (columns
// col0 .. col0 + cols of the vocabulary) update a running maximum m and a
// running sum s of exp(l - m) (online log-sum-exp, fp32), and record the
// label's logit when the label falls inside the chunk.
// zk_ce_bwd_chunk: overwrite the chunk with d loss / d logits =
// scale * (exp(l - lse) - [j == label]), rounded to the storage type.
// Rows whose label is negative (ignore_index) contribute nothing.
//
// One workgroup per row; each thread covers 8 consecutive columns per step
// (16-byte accesses for 2-byte types) and the row reductions use wave
// shuffles plus one LDS exchange.
#include "vec.h"

namespace zk {

template <int NT>
__device__ __forceinline__ void block_max_sum(float& m, float& s, float* red) {
  // combine (max, sum-of-exp relative to max) pairs across the workgroup
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float om = __shfl_xor(m, off, 64);
    const float os = __shfl_xor(s, off, 64);
    const float nm = fmaxf(m, om);
    s = (m == -INFINITY ? 0.f : s * expf(m - nm)) + (om == -INFINITY ? 0.f : os * expf(om - nm));
    m = nm;
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) {
    red[2 * wave] = m;
    red[2 * wave + 1] = s;
  }
  __syncthreads();
  m = -INFINITY;
  s = 0.f;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    const float om = red[2 * w], os = red[2 * w + 1];
    const float nm = fmaxf(m, om);
    s = (m == -INFINITY ? 0.f : s * expf(m - nm)) + (om == -INFINITY ? 0.f : os * expf(om - nm));
    m = nm;
  }
}

template <typename T, int NT>
__global__ __launch_bounds__(NT) void ce_fwd_chunk(const T* __restrict__ logits, int64_t cols,
                                                   int64_t ld, const int64_t* __restrict__ labels,
                                                   int64_t col0, float* __restrict__ run_max,
                                                   float* __restrict__ run_sum,
                                                   float* __restrict__ target) {
  __shared__ float red[2 * (NT / 64)];
  const int64_t row = blockIdx.x;
  const T* lr = logits + row * ld;
  const bool vec = (cols % 8) == 0;
  float m = -INFINITY, s = 0.f;
  if (vec) {
    for (int64_t c = threadIdx.x * 8; c < cols; c += NT * 8) {
      float v[8];
      Vec8<T>::load(lr + c, v);
      float lm = v[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) lm = fmaxf(lm, v[i]);
      const float nm = fmaxf(m, lm);
      float acc = m == -INFINITY ? 0.f : s * expf(m - nm);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc += expf(v[i] - nm);
      s = acc;
      m = nm;
    }
  } else {
    for (int64_t c = threadIdx.x; c < cols; c += NT) {
      const float v = to_f32(lr[c]);
      const float nm = fmaxf(m, v);
      s = (m == -INFINITY ? 0.f : s * expf(m - nm)) + expf(v - nm);
      m = nm;
    }
  }
  block_max_sum<NT>(m, s, red);
  if (threadIdx.x == 0) {
    const int64_t lab = labels[row];
    if (lab >= col0 && lab < col0 + cols) target[row] = to_f32(lr[lab - col0]);
    const float om = run_max[row], os = run_sum[row];
    const float nm = fmaxf(m, om);
    run_sum[row] = (m == -INFINITY ? 0.f : s * expf(m - nm)) +
                   (om == -INFINITY ? 0.f : os * expf(om - nm));
    run_max[row] = nm;
  }
}

template <typename T, int NT>
__global__ __launch_bounds__(NT) void ce_bwd_chunk(T* __restrict__ logits, int64_t cols, int64_t ld,
                                                   const int64_t* __restrict__ labels, int64_t col0,
                                                   const float* __restrict__ lse, float scale) {
  const int64_t row = blockIdx.x;
  T* lr = logits + row * ld;
  const int64_t lab = labels[row];
  const float l0 = lse[row];
  const float sc = lab < 0 ? 0.f : scale;
  if ((cols % 8) == 0) {
    for (int64_t c = threadIdx.x * 8; c < cols; c += NT * 8) {
      float v[8];
      Vec8<T>::load(lr + c, v);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        v[i] = lab < 0 ? 0.f : sc * (expf(v[i] - l0) - (col0 + c + i == lab ? 1.f : 0.f));
      Vec8<T>::store(lr + c, v);
    }
  } else {
    for (int64_t c = threadIdx.x; c < cols; c += NT) {
      const float v = to_f32(lr[c]);
      lr[c] = from_f32<T>(lab < 0 ? 0.f : sc * (expf(v - l0) - (col0 + c == lab ? 1.f : 0.f)));
    }
  }
}

}  // namespace zk

using namespace zk;

extern "C" int zk_ce_fwd_chunk(const void* logits, int64_t rows, int64_t cols, int64_t ld,
                               const int64_t* labels, int64_t col0, float* run_max,
                               float* run_sum, float* target_logit, int dtype,
                               zk_stream_t stream) {
  ZK_REQUIRE(valid_dtype(dtype), ZK_EDTYPE, "zk_ce_fwd_chunk: bad dtype %d", dtype);
  ZK_REQUIRE(rows >= 0 && cols > 0 && ld >= cols && col0 >= 0, ZK_EINVAL,
             "zk_ce_fwd_chunk: bad shape rows=%lld cols=%lld ld=%lld col0=%lld",
             (long long)rows, (long long)cols, (long long)ld, (long long)col0);
  ZK_REQUIRE(rows <= 0x7fffffff, ZK_EINVAL, "zk_ce_fwd_chunk: too many rows");
  if (rows == 0) return ZK_OK;
  ZK_REQUIRE(logits && labels && run_max && run_sum && target_logit, ZK_EINVAL,
             "zk_ce_fwd_chunk: null pointer");
  const bool vec_ok = cols % 8 == 0 && ld % 8 == 0 && aligned(logits, 16);
  ZK_REQUIRE(vec_ok || cols % 8 != 0, ZK_EALIGN,
             "zk_ce_fwd_chunk: logits must be 16-byte aligned with ld a multiple of 8");
  hipStream_t s = as_stream(stream);
  if (dtype == ZK_BF16)
    hipLaunchKernelGGL((ce_fwd_chunk<bf16, 256>), dim3(rows), dim3(256), 0, s, (const bf16*)logits,
                       cols, ld, labels, col0, run_max, run_sum, target_logit);
  else if (dtype == ZK_F16)
    hipLaunchKernelGGL((ce_fwd_chunk<f16, 256>), dim3(rows), dim3(256), 0, s, (const f16*)logits,
                       cols, ld, labels, col0, run_max, run_sum, target_logit);
  else
    hipLaunchKernelGGL((ce_fwd_chunk<float, 256>), dim3(rows), dim3(256), 0, s,
                       (const float*)logits, cols, ld, labels, col0, run_max, run_sum,
                       target_logit);
  return launch_status("zk_ce_fwd_chunk");
}

extern "C" int zk_ce_bwd_chunk(void* logits, int64_t rows, int64_t cols, int64_t ld,
                               const int64_t* labels, int64_t col0, const float* lse,
                               float scale, int dtype, zk_stream_t stream) {
  ZK_REQUIRE(valid_dtype(dtype), ZK_EDTYPE, "zk_ce_bwd_chunk: bad dtype %d", dtype);
  ZK_REQUIRE(rows >= 0 && cols > 0 && ld >= cols && col0 >= 0, ZK_EINVAL,
             "zk_ce_bwd_chunk: bad shape rows=%lld cols=%lld ld=%lld col0=%lld",
             (long long)rows, (long long)cols, (long long)ld, (long long)col0);
  ZK_REQUIRE(rows <= 0x7fffffff, ZK_EINVAL, "zk_ce_bwd_chunk: too many rows");
  if (rows == 0) return ZK_OK;
  ZK_REQUIRE(logits && labels && lse, ZK_EINVAL, "zk_ce_bwd_chunk: null pointer");
  const bool vec_ok = cols % 8 == 0 && ld % 8 == 0 && aligned(logits, 16);
  ZK_REQUIRE(vec_ok || cols % 8 != 0, ZK_EALIGN,
             "zk_ce_bwd_chunk: logits must be 16-byte aligned with ld a multiple of 8");
  hipStream_t s = as_stream(stream);
  if (dtype == ZK_BF16)
    hipLaunchKernelGGL((ce_bwd_chunk<bf16, 256>), dim3(rows), dim3(256), 0, s, (bf16*)logits,
                       cols, ld, labels, col0, lse, scale);
  else if (dtype == ZK_F16)
    hipLaunchKernelGGL((ce_bwd_chunk<f16, 256>), dim3(rows), dim3(256), 0, s, (f16*)logits,
                       cols, ld, labels, col0, lse, scale);
  else
    hipLaunchKernelGGL((ce_bwd_chunk<float, 256>), dim3(rows), dim3(256), 0, s, (float*)logits,
                       cols, ld, labels, col0, lse, scale);
  return launch_status("zk_ce_bwd_chunk");
}
