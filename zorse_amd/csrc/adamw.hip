// Fused AdamW step on one flat fp32 parameter shard.
//
// One pass over HBM: read p, g, m, v; write p, m, v (and the low-precision
// compute copy of p when requested).  28 bytes per element with an fp32
// grad, 26 with a bf16/fp16 grad, +2 for the low-precision copy.
//
// The flat kernel accesses every stream one element per lane (4-byte, or
// 2-byte for 16-bit types, accesses; 256 consecutive bytes of fp32 per wave
// and instruction).  Measured on gfx950 over a 202M-element shard (ordinary
// accesses), one element per thread ran at 78 % of the HBM peak, two at 72 %
// and four or eight (16-byte accesses per lane) at 66-68 %; with nontemporal
// accesses the one-element form reaches 82 %.  The region kernel below
// keeps 16-byte accesses: its one-element-per-lane form was slower alone
// (63-64 %) and, run beside the attention backward as the stage runs it,
// cost 2.3 ms per 8-layer step.
#include <cmath>

#include "zk_common.h"

namespace zk {

struct AdamScalars {
  float decay;         // 1 - lr * weight_decay
  float one_minus_b1;  // lerp weight of the first moment
  float b2, one_minus_b2;
  float step_size;     // lr / (1 - b1^t)
  float bc2_sqrt;      // sqrt(1 - b2^t)
  float eps;
};

template <typename G>
__device__ __forceinline__ void load_grad4(const G* g, int64_t i, float (&o)[4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = to_f32(g[i + k]);
}
template <>
__device__ __forceinline__ void load_grad4<float>(const float* g, int64_t i,
                                                  float (&o)[4]) {
  const float4 a = *reinterpret_cast<const float4*>(g + i);
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
}
template <>
__device__ __forceinline__ void load_grad4<bf16>(const bf16* g, int64_t i,
                                                 float (&o)[4]) {
  const bf16x4 a = *reinterpret_cast<const bf16x4*>(g + i);
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = static_cast<float>(a[k]);
}
template <>
__device__ __forceinline__ void load_grad4<f16>(const f16* g, int64_t i,
                                                float (&o)[4]) {
  const f16x4 a = *reinterpret_cast<const f16x4*>(g + i);
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = static_cast<float>(a[k]);
}

template <typename L>
__device__ __forceinline__ void store4(L* dst, const float4& v) {
  dst[0] = from_f32<L>(v.x); dst[1] = from_f32<L>(v.y);
  dst[2] = from_f32<L>(v.z); dst[3] = from_f32<L>(v.w);
}
template <>
__device__ __forceinline__ void store4<bf16>(bf16* dst, const float4& v) {
  bf16x4 a;
  a[0] = static_cast<bf16>(v.x); a[1] = static_cast<bf16>(v.y);
  a[2] = static_cast<bf16>(v.z); a[3] = static_cast<bf16>(v.w);
  *reinterpret_cast<bf16x4*>(dst) = a;
}
template <>
__device__ __forceinline__ void store4<f16>(f16* dst, const float4& v) {
  f16x4 a;
  a[0] = static_cast<f16>(v.x); a[1] = static_cast<f16>(v.y);
  a[2] = static_cast<f16>(v.z); a[3] = static_cast<f16>(v.w);
  *reinterpret_cast<f16x4*>(dst) = a;
}
template <>
__device__ __forceinline__ void store4<float>(float* dst, const float4& v) {
  *reinterpret_cast<float4*>(dst) = v;
}

__device__ __forceinline__ float adam_one(float& p, float g, float& m, float& v,
                                          const AdamScalars& s) {
  p = p * s.decay;
  m = fmaf(s.one_minus_b1, g - m, m);
  v = fmaf(s.one_minus_b2, g * g, v * s.b2);
  const float denom = sqrtf(v) / s.bc2_sqrt + s.eps;
  p = p - s.step_size * (m / denom);
  return p;
}

// 8 elements per thread (the region kernel): p, m, v as two 16-byte accesses
// each, the gradient and the low-precision copy as one 16-byte access for
// 2-byte types.
template <typename G>
__device__ __forceinline__ void load_grad8(const G* g, int64_t i, float (&o)[8]) {
  float a[4], b[4];
  load_grad4<G>(g, i, a);
  load_grad4<G>(g, i + 4, b);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    o[k] = a[k];
    o[k + 4] = b[k];
  }
}
template <>
__device__ __forceinline__ void load_grad8<bf16>(const bf16* g, int64_t i, float (&o)[8]) {
  const bf16x8 a = *reinterpret_cast<const bf16x8*>(g + i);
#pragma unroll
  for (int k = 0; k < 8; ++k) o[k] = static_cast<float>(a[k]);
}
template <>
__device__ __forceinline__ void load_grad8<f16>(const f16* g, int64_t i, float (&o)[8]) {
  const f16x8 a = *reinterpret_cast<const f16x8*>(g + i);
#pragma unroll
  for (int k = 0; k < 8; ++k) o[k] = static_cast<float>(a[k]);
}

template <typename L>
__device__ __forceinline__ void store8(L* dst, const float4& x, const float4& y) {
  store4<L>(dst, x);
  store4<L>(dst + 4, y);
}
template <>
__device__ __forceinline__ void store8<bf16>(bf16* dst, const float4& x, const float4& y) {
  const bf16x8 a = {static_cast<bf16>(x.x), static_cast<bf16>(x.y), static_cast<bf16>(x.z),
                    static_cast<bf16>(x.w), static_cast<bf16>(y.x), static_cast<bf16>(y.y),
                    static_cast<bf16>(y.z), static_cast<bf16>(y.w)};
  *reinterpret_cast<bf16x8*>(dst) = a;
}
template <>
__device__ __forceinline__ void store8<f16>(f16* dst, const float4& x, const float4& y) {
  const f16x8 a = {static_cast<f16>(x.x), static_cast<f16>(x.y), static_cast<f16>(x.z),
                   static_cast<f16>(x.w), static_cast<f16>(y.x), static_cast<f16>(y.y),
                   static_cast<f16>(y.z), static_cast<f16>(y.w)};
  *reinterpret_cast<f16x8*>(dst) = a;
}

// One element per thread, 256 consecutive elements per workgroup, no loop.
// L = float with kCopy = false means "no copy".  Every access is
// nontemporal: each element is touched once per step, so none of the 28 bytes
// is worth a place in L2 or the Infinity Cache.  Measured on a 202M-element
// shard: 0.865 ms (6.55 TB/s) against 0.90-0.91 ms with ordinary accesses,
// and the 7B stage, where the step runs beside the attention backward and
// the projection GEMMs, 41.70-41.84 ms/step against 42.38-42.41 (one process,
// alternating).
template <typename G, typename L, bool kCopy>
__global__ __launch_bounds__(256) void adamw_elem(float* __restrict__ p,
                                                  const G* __restrict__ g,
                                                  float* __restrict__ m,
                                                  float* __restrict__ v,
                                                  L* __restrict__ lowp, int64_t n,
                                                  AdamScalars s) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  float pv = __builtin_nontemporal_load(p + i), mv = __builtin_nontemporal_load(m + i),
        vv = __builtin_nontemporal_load(v + i);
  adam_one(pv, static_cast<float>(__builtin_nontemporal_load(g + i)), mv, vv, s);
  __builtin_nontemporal_store(pv, p + i);
  __builtin_nontemporal_store(mv, m + i);
  __builtin_nontemporal_store(vv, v + i);
  if (kCopy) {
    // round the stored fp32 value: left fused, the last fma would feed
    // v_fma_mix, which rounds the exact result to 16 bits in one step and
    // in rare cases differs from rounding the fp32 master
    asm volatile("" : "+v"(pv));
    __builtin_nontemporal_store(static_cast<L>(pv), lowp + i);
  }
}

// The same update over a shard described as row-major [rows, cols] regions
// (one launch per shard): for each region with a transposed-copy target the
// rounded parameter is also written transposed (lowp_t[c][r], row stride
// ld_t) -- the compute copy the backward's input-gradient GEMM reads along
// its reduction.  A workgroup owns a kTileR x kTileC tile of one region:
// 16-byte accesses on every stream (tile rows of kTileC elements), the
// rounded values staged in a padded LDS tile and written back as 16-byte
// chunks of 8 consecutive rows.  rows and cols are multiples of 8.
static constexpr int kMaxAdamRegions = 8;
struct AdamRegions {
  int64_t offset[kMaxAdamRegions];
  int64_t rows[kMaxAdamRegions];
  int64_t cols[kMaxAdamRegions];
  int64_t ld_t[kMaxAdamRegions];
  void* lowp_t[kMaxAdamRegions];
  int64_t tiles_x[kMaxAdamRegions];      // column tiles per region
  int64_t first_tile[kMaxAdamRegions + 1];  // prefix sums of the tile counts
  int n;
};

// tile of the region kernel: kTileR rows x kTileC columns per workgroup
static constexpr int kTileR = 64, kTileC = 128;

template <typename G, typename L>
__global__ __launch_bounds__(256) void adamw_tile_t(
    float* __restrict__ p, const G* __restrict__ g, float* __restrict__ m,
    float* __restrict__ v, L* __restrict__ lowp, AdamRegions reg, AdamScalars s) {
  constexpr int TR = kTileR, TC = kTileC;
  constexpr int CPR = TC / 8;              // 8-element chunks per tile row
  constexpr int NG = TR * CPR / 256;       // chunks per thread
  constexpr int RPP = 256 / CPR;           // tile rows per pass
  __shared__ L tile[TR][TC + 2];
  const int64_t bid = blockIdx.x;
  int ri = 0;
#pragma unroll
  for (int k = 1; k < kMaxAdamRegions; ++k)
    if (k < reg.n && bid >= reg.first_tile[k]) ri = k;
  const int64_t local = bid - reg.first_tile[ri];
  const int64_t rows = reg.rows[ri], cols = reg.cols[ri];
  const int64_t r0 = local / reg.tiles_x[ri] * TR;
  const int64_t c0 = local % reg.tiles_x[ri] * TC;
  const int64_t base = reg.offset[ri];
  const int tid = threadIdx.x;
  float4 pa[NG][2], ma[NG][2], va[NG][2];
  float gv[NG][8];
  bool in[NG];
#pragma unroll
  for (int k = 0; k < NG; ++k) {  // rows k * RPP + tid / CPR, columns 8 (tid % CPR)
    const int r = k * RPP + tid / CPR, ch = tid % CPR;
    const int64_t gr = r0 + r, gc = c0 + 8 * ch;
    in[k] = gr < rows && gc < cols;
    if (in[k]) {
      const int64_t i = base + gr * cols + gc;
      pa[k][0] = *reinterpret_cast<const float4*>(p + i);
      pa[k][1] = *reinterpret_cast<const float4*>(p + i + 4);
      ma[k][0] = *reinterpret_cast<const float4*>(m + i);
      ma[k][1] = *reinterpret_cast<const float4*>(m + i + 4);
      va[k][0] = *reinterpret_cast<const float4*>(v + i);
      va[k][1] = *reinterpret_cast<const float4*>(v + i + 4);
      load_grad8<G>(g, i, gv[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < NG; ++k) {
    if (!in[k]) continue;
    const int r = k * RPP + tid / CPR, ch = tid % CPR;
    const int64_t i = base + (r0 + r) * cols + c0 + 8 * ch;
    float4 &p0 = pa[k][0], &p1 = pa[k][1], &m0 = ma[k][0], &m1 = ma[k][1];
    float4 &v0 = va[k][0], &v1 = va[k][1];
    adam_one(p0.x, gv[k][0], m0.x, v0.x, s);
    adam_one(p0.y, gv[k][1], m0.y, v0.y, s);
    adam_one(p0.z, gv[k][2], m0.z, v0.z, s);
    adam_one(p0.w, gv[k][3], m0.w, v0.w, s);
    adam_one(p1.x, gv[k][4], m1.x, v1.x, s);
    adam_one(p1.y, gv[k][5], m1.y, v1.y, s);
    adam_one(p1.z, gv[k][6], m1.z, v1.z, s);
    adam_one(p1.w, gv[k][7], m1.w, v1.w, s);
    *reinterpret_cast<float4*>(p + i) = p0;
    *reinterpret_cast<float4*>(p + i + 4) = p1;
    *reinterpret_cast<float4*>(m + i) = m0;
    *reinterpret_cast<float4*>(m + i + 4) = m1;
    *reinterpret_cast<float4*>(v + i) = v0;
    *reinterpret_cast<float4*>(v + i + 4) = v1;
    store8<L>(lowp + i, p0, p1);
    const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[r][8 * ch + e] = static_cast<L>(pv[e]);
  }
  L* lt = static_cast<L*>(reg.lowp_t[ri]);
  if (lt == nullptr) return;  // region without a transposed copy (uniform)
  const int64_t ld_t = reg.ld_t[ri];
  __syncthreads();
  constexpr int RC = TR / 8;               // 8-row chunks per transposed row
#pragma unroll
  for (int k = 0; k < TC * RC / 256; ++k) {
    const int q = k * 256 + tid;
    const int c = q / RC, ch = q % RC;
    const int64_t gc = c0 + c, gr = r0 + 8 * ch;
    if (gc < cols && gr < rows) {
      typedef L L8 __attribute__((ext_vector_type(8)));
      L8 w;
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = tile[8 * ch + e][c];
      *reinterpret_cast<L8*>(lt + gc * ld_t + gr) = w;
    }
  }
}

template <typename G, typename L, bool kCopy>
static void launch_elem(float* p, const void* g, float* m, float* v, void* lowp, int64_t n,
                        const AdamScalars& s, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((n + 255) / 256));
  hipLaunchKernelGGL((adamw_elem<G, L, kCopy>), grid, dim3(256), 0, st, p,
                     static_cast<const G*>(g), m, v, static_cast<L*>(lowp), n, s);
}

template <typename G>
static void launch_flat(float* p, const void* g, float* m, float* v, void* lowp, int ldt,
                        int64_t n, const AdamScalars& s, hipStream_t st) {
  if (lowp == nullptr) launch_elem<G, float, false>(p, g, m, v, nullptr, n, s, st);
  else if (ldt == ZK_BF16) launch_elem<G, bf16, true>(p, g, m, v, lowp, n, s, st);
  else if (ldt == ZK_F16) launch_elem<G, f16, true>(p, g, m, v, lowp, n, s, st);
  else launch_elem<G, float, true>(p, g, m, v, lowp, n, s, st);
}

static AdamScalars adam_scalars(double lr, double beta1, double beta2, double eps,
                                double weight_decay, int64_t step) {
  AdamScalars s;
  s.decay = static_cast<float>(1.0 - lr * weight_decay);
  s.one_minus_b1 = static_cast<float>(1.0 - beta1);
  s.b2 = static_cast<float>(beta2);
  s.one_minus_b2 = static_cast<float>(1.0 - beta2);
  const double bc1 = 1.0 - std::pow(beta1, static_cast<double>(step));
  const double bc2 = 1.0 - std::pow(beta2, static_cast<double>(step));
  s.step_size = static_cast<float>(lr / bc1);
  s.bc2_sqrt = static_cast<float>(std::sqrt(bc2));
  s.eps = static_cast<float>(eps);
  return s;
}

}  // namespace zk

using namespace zk;

extern "C" int zk_adamw_step(float* param, const void* grad, int grad_dtype,
                             float* exp_avg, float* exp_avg_sq,
                             void* param_lowp, int lowp_dtype, int64_t n,
                             double lr, double beta1, double beta2, double eps,
                             double weight_decay, int64_t step,
                             zk_stream_t stream) {
  ZK_REQUIRE(valid_dtype(grad_dtype), ZK_EDTYPE,
             "zk_adamw_step: bad grad dtype %d", grad_dtype);
  ZK_REQUIRE(param_lowp == nullptr || valid_dtype(lowp_dtype), ZK_EDTYPE,
             "zk_adamw_step: bad low-precision dtype %d", lowp_dtype);
  ZK_REQUIRE(n >= 0, ZK_EINVAL, "zk_adamw_step: negative n");
  ZK_REQUIRE(step >= 1, ZK_EINVAL, "zk_adamw_step: step must be >= 1 (got %lld)",
             (long long)step);
  ZK_REQUIRE(n == 0 || (param && grad && exp_avg && exp_avg_sq), ZK_EINVAL,
             "zk_adamw_step: null pointer");
  ZK_REQUIRE(lr >= 0 && beta1 >= 0 && beta1 < 1 && beta2 >= 0 && beta2 < 1 &&
                 eps >= 0 && weight_decay >= 0,
             ZK_EINVAL, "zk_adamw_step: hyper-parameter out of range");
  if (n == 0) return ZK_OK;
  const AdamScalars s = adam_scalars(lr, beta1, beta2, eps, weight_decay, step);

  ZK_REQUIRE(aligned(param, 4) && aligned(exp_avg, 4) && aligned(exp_avg_sq, 4) &&
                 aligned(grad, dtype_bytes(grad_dtype)) &&
                 (param_lowp == nullptr || aligned(param_lowp, dtype_bytes(lowp_dtype))),
             ZK_EALIGN, "zk_adamw_step: operands must be aligned to their element size");
  ZK_REQUIRE((n + 255) / 256 <= 0x7fffffffLL, ZK_EINVAL, "zk_adamw_step: shard too large (%lld)",
             (long long)n);
  hipStream_t st = as_stream(stream);
  if (grad_dtype == ZK_F32)
    launch_flat<float>(param, grad, exp_avg, exp_avg_sq, param_lowp, lowp_dtype, n, s, st);
  else if (grad_dtype == ZK_BF16)
    launch_flat<bf16>(param, grad, exp_avg, exp_avg_sq, param_lowp, lowp_dtype, n, s, st);
  else
    launch_flat<f16>(param, grad, exp_avg, exp_avg_sq, param_lowp, lowp_dtype, n, s, st);
  return launch_status("zk_adamw_step");
}

extern "C" int zk_adamw_step_t(float* param, const void* grad, int grad_dtype, float* exp_avg,
                               float* exp_avg_sq, void* param_lowp, int lowp_dtype,
                               const zk_adamw_region* regions, int n_regions, int64_t n,
                               double lr, double beta1, double beta2, double eps,
                               double weight_decay, int64_t step, zk_stream_t stream) {
  ZK_REQUIRE(valid_dtype(grad_dtype), ZK_EDTYPE, "zk_adamw_step_t: bad grad dtype %d",
             grad_dtype);
  ZK_REQUIRE(lowp_dtype == ZK_BF16 || lowp_dtype == ZK_F16, ZK_EDTYPE,
             "zk_adamw_step_t: the compute copy must be bf16 or fp16 (got %d)", lowp_dtype);
  ZK_REQUIRE(n_regions >= 0 && n_regions <= kMaxAdamRegions, ZK_EINVAL,
             "zk_adamw_step_t: 0 .. %d regions (got %d)", kMaxAdamRegions, n_regions);
  ZK_REQUIRE(n_regions == 0 || regions != nullptr, ZK_EINVAL, "zk_adamw_step_t: null regions");
  ZK_REQUIRE(step >= 1, ZK_EINVAL, "zk_adamw_step_t: step must be >= 1 (got %lld)",
             (long long)step);
  ZK_REQUIRE(lr >= 0 && beta1 >= 0 && beta1 < 1 && beta2 >= 0 && beta2 < 1 &&
                 eps >= 0 && weight_decay >= 0,
             ZK_EINVAL, "zk_adamw_step_t: hyper-parameter out of range");
  AdamRegions reg = {};
  int64_t tiles = 0, prev_end = 0;
  for (int i = 0; i < n_regions; ++i) {
    const zk_adamw_region& r = regions[i];
    ZK_REQUIRE(r.offset >= prev_end && r.rows >= 0 && r.cols >= 0, ZK_EINVAL,
               "zk_adamw_step_t: region %d overlaps or has a bad shape", i);
    ZK_REQUIRE(r.offset % 8 == 0 && r.rows % 8 == 0 && r.cols % 8 == 0, ZK_EUNSUPPORTED,
               "zk_adamw_step_t: region %d: offset, rows and cols must be multiples of 8", i);
    ZK_REQUIRE(r.lowp_t == nullptr || (r.ld_t >= r.rows && r.ld_t % 8 == 0 && aligned(r.lowp_t, 16)),
               ZK_EALIGN, "zk_adamw_step_t: region %d: bad transposed target", i);
    ZK_REQUIRE((r.rows + kTileR - 1) / kTileR * ((r.cols + kTileC - 1) / kTileC) < 0x40000000LL, ZK_EINVAL,
               "zk_adamw_step_t: region %d too large", i);
    reg.offset[i] = r.offset;
    reg.rows[i] = r.rows;
    reg.cols[i] = r.cols;
    reg.ld_t[i] = r.ld_t;
    reg.lowp_t[i] = r.lowp_t;
    const int64_t tx = (r.cols + kTileC - 1) / kTileC, ty = (r.rows + kTileR - 1) / kTileR;
    reg.tiles_x[i] = tx > 0 ? tx : 1;
    reg.first_tile[i] = tiles;
    tiles += tx * ty;
    prev_end = r.offset + r.rows * r.cols;
    ZK_REQUIRE(prev_end <= n, ZK_EINVAL,
               "zk_adamw_step_t: region %d ends at %lld, past the shard's %lld elements", i,
               (long long)prev_end, (long long)n);
  }
  reg.first_tile[n_regions] = tiles;
  reg.n = n_regions;
  if (tiles == 0) return ZK_OK;
  ZK_REQUIRE(tiles < 0x7fffffffLL, ZK_EINVAL, "zk_adamw_step_t: shard too large");
  const void* ptrs[] = {param, grad, exp_avg, exp_avg_sq, param_lowp};
  for (const void* p : ptrs) {
    ZK_REQUIRE(p != nullptr, ZK_EINVAL, "zk_adamw_step_t: null pointer");
    ZK_REQUIRE(aligned(p, 16), ZK_EALIGN, "zk_adamw_step_t: operands must be 16-byte aligned");
  }
  const AdamScalars s = adam_scalars(lr, beta1, beta2, eps, weight_decay, step);
  hipStream_t st = as_stream(stream);
  const dim3 grid(static_cast<unsigned>(tiles));
#define ZK_T(G, L)                                                                          \
  hipLaunchKernelGGL((adamw_tile_t<G, L>), grid, dim3(256), 0, st, param, (const G*)grad,  \
                     exp_avg, exp_avg_sq, (L*)param_lowp, reg, s)
  if (lowp_dtype == ZK_BF16) {
    if (grad_dtype == ZK_BF16) ZK_T(bf16, bf16);
    else if (grad_dtype == ZK_F16) ZK_T(f16, bf16);
    else ZK_T(float, bf16);
  } else {
    if (grad_dtype == ZK_BF16) ZK_T(bf16, f16);
    else if (grad_dtype == ZK_F16) ZK_T(f16, f16);
    else ZK_T(float, f16);
  }
#undef ZK_T
  return launch_status("zk_adamw_step_t");
}
