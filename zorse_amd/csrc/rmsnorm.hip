// RMSNorm forward / backward for gfx950.
//
// Vector kernels: NT threads x CH chunks of 8 elements per row (16-byte
// accesses for 2-byte types), CH a compile-time constant so a row lives in
// exactly CH x 8 registers per thread.  The forward runs one workgroup per
// row: x is read once and y written once, the HBM minimum.  The backward
// walks rows in groups of kBwdRows with a grid of at most kBwdParts
// workgroups: the group's dy, h (and residual gradient) loads are all issued
// before its row reductions (for 2-byte rows of up to 4096 elements also the
// next group's, while this one is processed); the row sums share one pair of
// barriers, each thread accumulates the weight gradient of its fixed columns in registers,
// and every workgroup writes one fp32 partial row that a second kernel
// reduces deterministically (no atomics).  Rows whose width is not a
// multiple of 8, wider than 8192, or misaligned buffers take the scalar
// kernels, which read the row twice.
#include <mutex>

#include "vec.h"

namespace zk {

static constexpr int kBwdParts = 512;  // workgroups (= dw partial rows) of the backward
static constexpr int kBwdRows = 2;     // rows a backward workgroup keeps in flight
static constexpr int kMaxCh = 4;       // chunks of 8 per thread: hidden <= 256 * 4 * 8

template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (NT > 64) {
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) t += red[i];
    __syncthreads();
    return t;
  }
  return v;
}

// ---------------------------------------------------------------- forward ---
template <typename T, typename W, int NT, int CH>
__global__ __launch_bounds__(NT) void rmsnorm_fwd_vec(
    const T* __restrict__ x, const T* __restrict__ res, T* __restrict__ hout,
    const W* __restrict__ w, T* __restrict__ y, float* __restrict__ rstd,
    int64_t hidden, float eps) {
  __shared__ float red[NT / 64];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * hidden;
  const int nchunk = static_cast<int>(hidden / 8);
  // every load of the row (and of its residual) first, in storage format, so
  // that all of them are in flight together; widened afterwards
  Raw8<T> xraw[CH], rraw[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = threadIdx.x + c * NT;
    if (ch < nchunk) xraw[c].load(xr + ch * 8);
  }
  if (res != nullptr) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int ch = threadIdx.x + c * NT;
      if (ch < nchunk) rraw[c].load(res + row * hidden + ch * 8);
    }
  }
  float v[CH][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = threadIdx.x + c * NT;
    if (ch < nchunk) {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[c][i] = xraw[c][i];
      if (res != nullptr) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[c][i] = round_to<T>(v[c][i] + rraw[c][i]);
        Vec8<T>::store(hout + row * hidden + ch * 8, v[c]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(v[c][i], v[c][i], ss);
    }
  }
  ss = block_sum<NT>(ss, red);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(hidden) + eps);
  if (threadIdx.x == 0) rstd[row] = r;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = threadIdx.x + c * NT;
    if (ch < nchunk) {
      float w8[8], o[8];
      Vec8<W>::load(w + ch * 8, w8);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = w8[i] * round_to<T>(v[c][i] * r);
      Vec8<T>::store(y + row * hidden + ch * 8, o);
    }
  }
}

// Scalar fallback: any width / alignment; dtypes by runtime code.
__global__ __launch_bounds__(256) void rmsnorm_fwd_scalar(
    const void* __restrict__ x, const void* __restrict__ res,
    void* __restrict__ hout, const void* __restrict__ w, void* __restrict__ y,
    float* __restrict__ rstd, int64_t hidden, float eps, int adt, int wdt) {
  __shared__ float red[4];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * hidden;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < hidden; i += 256) {
    float h = load_dt(x, base + i, adt);
    if (res != nullptr) {
      h = h + load_dt(res, base + i, adt);
      store_dt(hout, base + i, adt, h);
      h = load_dt(hout, base + i, adt);  // rounded value
    }
    ss = fmaf(h, h, ss);
  }
  ss = block_sum<256>(ss, red);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(hidden) + eps);
  if (threadIdx.x == 0) rstd[blockIdx.x] = r;
  const void* src = res != nullptr ? hout : x;
  for (int64_t i = threadIdx.x; i < hidden; i += 256) {
    const float h = load_dt(src, base + i, adt);
    float xh = h * r;
    if (adt != ZK_F32) xh = adt == ZK_BF16 ? round_to<bf16>(xh) : round_to<f16>(xh);
    store_dt(y, base + i, adt, load_dt(w, i, wdt) * xh);
  }
}

// --------------------------------------------------------------- backward ---
// R rows are processed together: all their loads are issued before the
// first reduction, and the R row sums share one pair of barriers, so a
// workgroup keeps R rows of dy and h in flight.
template <int NT, int R>
__device__ __forceinline__ void block_sum_rows(float (&v)[R], float* red) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < R; ++r) v[r] = wave_sum(v[r]);
  if (NT > 64) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r) red[r * (NT / 64) + wave] = v[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < NT / 64; ++i) t += red[r * (NT / 64) + i];
      v[r] = t;
    }
    __syncthreads();
  }
}

// The rows of one group (dy, h, dres) in packed form plus their rstd.
template <typename T, int R, int CH, bool kRes>
struct BwdGroup {
  Raw8<T> d8[R][CH], h8[R][CH], g8[kRes ? R : 1][CH];
  float r[R];
};

template <typename T, typename W, int NT, int R, int CH, bool kRes>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2)))
void rmsnorm_bwd_vec(
    const T* __restrict__ dy, const T* __restrict__ h, const W* __restrict__ w,
    const float* __restrict__ rstd, const T* __restrict__ dres,
    T* __restrict__ dx, float* __restrict__ part, int64_t rows,
    int64_t hidden) {
  typedef BwdGroup<T, R, CH, kRes> G;
  __shared__ float red[R * (NT / 64)];
  const int nchunk = static_cast<int>(hidden / 8);
  float wv[CH][8], dw[CH][8];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = threadIdx.x + c * NT;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      dw[c][i] = 0.f;
      wv[c][i] = 0.f;
    }
    if (ch < nchunk) Vec8<W>::load(w + ch * 8, wv[c]);
  }

  auto load = [&](G& gr, int64_t row0) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int64_t row = row0 + k < rows ? row0 + k : rows - 1;
      gr.r[k] = row0 + k < rows ? rstd[row] : 0.f;  // r = 0: the row contributes nothing
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int ch = threadIdx.x + c * NT;
        if (ch < nchunk) {
          gr.d8[k][c].load(dy + row * hidden + ch * 8);
          gr.h8[k][c].load(h + row * hidden + ch * 8);
          if (kRes) gr.g8[kRes ? k : 0][c].load(dres + row * hidden + ch * 8);
        } else {
          gr.d8[k][c].zero();
          gr.h8[k][c].zero();
        }
      }
    }
  };

  auto process = [&](G& gr, int64_t row0) __attribute__((always_inline)) {
    float dot[R];
#pragma unroll
    for (int k = 0; k < R; ++k) {
      dot[k] = 0.f;
#pragma unroll
      for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float xh = gr.h8[k][c][i] * gr.r[k];
          dot[k] = fmaf(gr.d8[k][c][i] * wv[c][i], xh, dot[k]);
          dw[c][i] = fmaf(gr.d8[k][c][i], round_to<T>(xh), dw[c][i]);
        }
    }
    block_sum_rows<NT, R>(dot, red);
#pragma unroll
    for (int k = 0; k < R; ++k)
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        gr.d8[k][c].opaque();
        gr.h8[k][c].opaque();
      }
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int64_t row = row0 + k;
      if (row >= rows) break;
      const float mean = dot[k] / static_cast<float>(hidden);
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int ch = threadIdx.x + c * NT;
        if (ch < nchunk) {
          float o[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float xh = gr.h8[k][c][i] * gr.r[k];
            o[i] = gr.r[k] * (gr.d8[k][c][i] * wv[c][i] - xh * mean);
            if (kRes) o[i] += gr.g8[kRes ? k : 0][c][i];
          }
          Vec8<T>::store(dx + row * hidden + ch * 8, o);
        }
      }
    }
  };

  // Row groups blockIdx.x, + gridDim.x, ...  For 2-byte rows of up to 2
  // chunks per thread the next group's loads are in flight while the current
  // one is reduced and written (two buffers, alternated by unrolling the loop
  // by two); wider rows have no registers for a second buffer.
  const int64_t stride = static_cast<int64_t>(gridDim.x) * R;
  int64_t row0 = static_cast<int64_t>(blockIdx.x) * R;
  if constexpr (CH <= 2 && sizeof(T) == 2) {
    G ga, gb;
    if (row0 < rows) load(ga, row0);
    while (row0 < rows) {
      int64_t nxt = row0 + stride;
      if (nxt < rows) load(gb, nxt);
      process(ga, row0);
      row0 = nxt;
      if (row0 >= rows) break;
      nxt = row0 + stride;
      if (nxt < rows) load(ga, nxt);
      process(gb, row0);
      row0 = nxt;
    }
  } else {
    for (; row0 < rows; row0 += stride) {
      G ga;
      load(ga, row0);
      process(ga, row0);
    }
  }
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = threadIdx.x + c * NT;
    if (ch < nchunk)
      Vec8<float>::store(part + static_cast<int64_t>(blockIdx.x) * hidden + ch * 8,
                         dw[c]);
  }
}

__global__ __launch_bounds__(256) void rmsnorm_bwd_scalar(
    const void* __restrict__ dy, const void* __restrict__ h,
    const void* __restrict__ w, const float* __restrict__ rstd,
    const void* __restrict__ dres, void* __restrict__ dx,
    float* __restrict__ part, int64_t rows, int64_t hidden, int adt,
    int wdt) {
  __shared__ float red[4];
  float* prow = part + static_cast<int64_t>(blockIdx.x) * hidden;
  for (int64_t i = threadIdx.x; i < hidden; i += 256) prow[i] = 0.f;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const int64_t base = row * hidden;
    const float r = rstd[row];
    float dot = 0.f;
    for (int64_t i = threadIdx.x; i < hidden; i += 256) {
      const float xh = load_dt(h, base + i, adt) * r;
      const float d = load_dt(dy, base + i, adt);
      dot = fmaf(d * load_dt(w, i, wdt), xh, dot);
      float xr = xh;
      if (adt != ZK_F32) xr = adt == ZK_BF16 ? round_to<bf16>(xh) : round_to<f16>(xh);
      prow[i] = fmaf(d, xr, prow[i]);
    }
    dot = block_sum<256>(dot, red);
    const float mean = dot / static_cast<float>(hidden);
    for (int64_t i = threadIdx.x; i < hidden; i += 256) {
      const float xh = load_dt(h, base + i, adt) * r;
      const float g = load_dt(dy, base + i, adt) * load_dt(w, i, wdt);
      float o = r * (g - xh * mean);
      if (dres != nullptr) o += load_dt(dres, base + i, adt);
      store_dt(dx, base + i, adt, o);
    }
  }
}

// dw[c] = sum_p part[p][c]  (optionally added to the existing dw).  A
// workgroup owns 64 columns; its 16 waves stride over the partial rows with 4
// independent running sums each and meet in LDS.  nparts == 0 writes zeros
// (or leaves dw unchanged).  (16 columns per workgroup, which spreads the
// reduction over every CU, read the partial rows in 64-byte segments: 8 %
// more HBM traffic for the whole backward and no gain in time.)
__global__ __launch_bounds__(1024) void rmsnorm_dw_reduce(
    const float* __restrict__ part, int64_t nparts, int64_t hidden,
    void* __restrict__ dw, int wdt, int accumulate) {
  __shared__ float red[16][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  if (c < hidden) {
    int64_t p = wave;
    for (; p + 48 < nparts; p += 64) {
      s0 += part[p * hidden + c];
      s1 += part[(p + 16) * hidden + c];
      s2 += part[(p + 32) * hidden + c];
      s3 += part[(p + 48) * hidden + c];
    }
    for (; p < nparts; p += 16) s0 += part[p * hidden + c];
  }
  red[wave][lane] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  if (wave == 0 && c < hidden) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) t += red[i][lane];
    if (accumulate) t += load_dt(dw, c, wdt);
    store_dt(dw, c, wdt, t);
  }
}

// ------------------------------------------------------------ dispatch ------
// Threads per row and chunks per thread for a row of `hidden` elements.
static void pick_shape(int64_t hidden, int& nt, int& ch) {
  const int64_t nchunk = hidden / 8;
  nt = nchunk <= 64 ? 64 : nchunk <= 128 ? 128 : 256;
  ch = static_cast<int>((nchunk + nt - 1) / nt);
}

template <typename T, typename W>
static void launch_fwd_vec(const void* x, const void* res, void* hout,
                           const void* w, void* y, float* rstd, int64_t rows,
                           int64_t hidden, float eps, hipStream_t s) {
  int nt, ch;
  pick_shape(hidden, nt, ch);
  // The forward keeps one row per workgroup: prefer 128 threads x up to 4
  // chunks (more bytes in flight per thread, more workgroups per CU).  At
  // 4096 x 4096 bf16 (one box, rotating buffers): 12.0 us with the kernel's
  // loads issued before any math, 12.9 for one wave x 8 chunks, 13.0 for
  // this shape with each chunk's math right after its load.
  const int64_t nchunk = hidden / 8;
  if (nt == 256 && nchunk <= 128 * kMaxCh) {
    nt = 128;
    ch = static_cast<int>((nchunk + 127) / 128);
  }
#define ZK_LAUNCH(NT, CH)                                                          \
  hipLaunchKernelGGL((rmsnorm_fwd_vec<T, W, NT, CH>), dim3(rows), dim3(NT), 0, s,  \
                     (const T*)x, (const T*)res, (T*)hout, (const W*)w, (T*)y, rstd, \
                     hidden, eps)
  if (nt == 64) ZK_LAUNCH(64, 1);
  else if (nt == 128 && ch == 1) ZK_LAUNCH(128, 1);
  else if (nt == 128 && ch == 2) ZK_LAUNCH(128, 2);
  else if (nt == 128 && ch == 3) ZK_LAUNCH(128, 3);
  else if (nt == 128) ZK_LAUNCH(128, 4);
  else if (ch == 1) ZK_LAUNCH(256, 1);
  else if (ch == 2) ZK_LAUNCH(256, 2);
  else if (ch == 3) ZK_LAUNCH(256, 3);
  else ZK_LAUNCH(256, 4);
#undef ZK_LAUNCH
}

template <typename T, typename W, bool kRes>
static void launch_bwd_vec_r(const void* dy, const void* h, const void* w,
                             const float* rstd, const void* dres, void* dx,
                             float* part, int64_t nparts, int64_t rows,
                             int64_t hidden, hipStream_t s) {
  int nt, ch;
  pick_shape(hidden, nt, ch);
#define ZK_LAUNCH(NT, CH)                                                          \
  hipLaunchKernelGGL((rmsnorm_bwd_vec<T, W, NT, kBwdRows, CH, kRes>), dim3(nparts), \
                     dim3(NT), 0, s, (const T*)dy, (const T*)h, (const W*)w, rstd,  \
                     (const T*)dres, (T*)dx, part, rows, hidden)
  if (nt == 64) ZK_LAUNCH(64, 1);
  else if (nt == 128) ZK_LAUNCH(128, 1);
  else if (ch == 1) ZK_LAUNCH(256, 1);
  else if (ch == 2) ZK_LAUNCH(256, 2);
  else if (ch == 3) ZK_LAUNCH(256, 3);
  else ZK_LAUNCH(256, 4);
#undef ZK_LAUNCH
}

template <typename T, typename W>
static void launch_bwd_vec(const void* dy, const void* h, const void* w,
                           const float* rstd, const void* dres, void* dx,
                           float* part, int64_t nparts, int64_t rows,
                           int64_t hidden, hipStream_t s) {
  if (dres != nullptr)
    launch_bwd_vec_r<T, W, true>(dy, h, w, rstd, dres, dx, part, nparts, rows, hidden, s);
  else
    launch_bwd_vec_r<T, W, false>(dy, h, w, rstd, dres, dx, part, nparts, rows, hidden, s);
}

template <typename T>
static bool dispatch_w_fwd(int wdt, const void* x, const void* res, void* hout,
                           const void* w, void* y, float* rstd, int64_t rows,
                           int64_t hidden, float eps, hipStream_t s) {
  if (wdt == ZK_F32) launch_fwd_vec<T, float>(x, res, hout, w, y, rstd, rows, hidden, eps, s);
  else if (wdt == ZK_BF16) launch_fwd_vec<T, bf16>(x, res, hout, w, y, rstd, rows, hidden, eps, s);
  else launch_fwd_vec<T, f16>(x, res, hout, w, y, rstd, rows, hidden, eps, s);
  return true;
}

template <typename T>
static void dispatch_w_bwd(int wdt, const void* dy, const void* h,
                           const void* w, const float* rstd, const void* dres,
                           void* dx, float* part, int64_t nparts, int64_t rows,
                           int64_t hidden, hipStream_t s) {
  if (wdt == ZK_F32) launch_bwd_vec<T, float>(dy, h, w, rstd, dres, dx, part, nparts, rows, hidden, s);
  else if (wdt == ZK_BF16) launch_bwd_vec<T, bf16>(dy, h, w, rstd, dres, dx, part, nparts, rows, hidden, s);
  else launch_bwd_vec<T, f16>(dy, h, w, rstd, dres, dx, part, nparts, rows, hidden, s);
}

static bool vec_ok(int64_t hidden, int adt, int wdt,
                   std::initializer_list<const void*> ptrs) {
  if (hidden % 8 != 0 || hidden / 8 > 256 * kMaxCh) return false;  // hidden <= 8192
  for (const void* p : ptrs)
    if (p != nullptr && !aligned(p, 16)) return false;
  (void)adt;
  (void)wdt;
  return true;
}

}  // namespace zk

using namespace zk;

extern "C" int zk_rmsnorm_fwd(const void* x, const void* residual, void* h_out,
                              const void* w, void* y, float* rstd, int64_t rows,
                              int64_t hidden, float eps, int act_dtype,
                              int w_dtype, zk_stream_t stream) {
  ZK_REQUIRE(valid_dtype(act_dtype) && valid_dtype(w_dtype), ZK_EDTYPE,
             "zk_rmsnorm_fwd: bad dtype code (%d, %d)", act_dtype, w_dtype);
  ZK_REQUIRE(rows >= 0 && hidden > 0, ZK_EINVAL,
             "zk_rmsnorm_fwd: bad shape rows=%lld hidden=%lld",
             (long long)rows, (long long)hidden);
  ZK_REQUIRE(x && w && y && rstd, ZK_EINVAL, "zk_rmsnorm_fwd: null pointer");
  ZK_REQUIRE(residual == nullptr || h_out != nullptr, ZK_EINVAL,
             "zk_rmsnorm_fwd: residual given without h_out");
  ZK_REQUIRE(rows <= 0x7fffffff, ZK_EINVAL, "zk_rmsnorm_fwd: too many rows");
  if (rows == 0) return ZK_OK;
  hipStream_t s = as_stream(stream);
  if (vec_ok(hidden, act_dtype, w_dtype, {x, residual, h_out, w, y})) {
    if (act_dtype == ZK_BF16) dispatch_w_fwd<bf16>(w_dtype, x, residual, h_out, w, y, rstd, rows, hidden, eps, s);
    else if (act_dtype == ZK_F16) dispatch_w_fwd<f16>(w_dtype, x, residual, h_out, w, y, rstd, rows, hidden, eps, s);
    else dispatch_w_fwd<float>(w_dtype, x, residual, h_out, w, y, rstd, rows, hidden, eps, s);
  } else {
    hipLaunchKernelGGL(rmsnorm_fwd_scalar, dim3(rows), dim3(256), 0, s, x,
                       residual, h_out, w, y, rstd, hidden, eps, act_dtype,
                       w_dtype);
  }
  return launch_status("zk_rmsnorm_fwd");
}

extern "C" int64_t zk_rmsnorm_bwd_workspace(int64_t rows, int64_t hidden) {
  if (rows <= 0 || hidden <= 0) return 0;
  const int64_t groups = (rows + kBwdRows - 1) / kBwdRows;
  const int64_t parts = groups < kBwdParts ? groups : kBwdParts;
  return parts * hidden;
}

namespace zk {

// The backward of both entry points, with the dw partial rows in `workspace`
// (workspace_elems floats, at least zk_rmsnorm_bwd_workspace(rows, hidden)).
// Every launched workgroup writes its whole partial row before the reduction
// reads it, so the workspace needs no clearing.
static int rmsnorm_bwd_impl(const char* who, const void* dy, const void* h, const void* w,
                            const float* rstd, const void* dres, void* dx, void* dw,
                            int accumulate, float* workspace, int64_t workspace_elems,
                            int64_t rows, int64_t hidden, int act_dtype, int w_dtype,
                            hipStream_t s) {
  const int64_t need = zk_rmsnorm_bwd_workspace(rows, hidden);
  ZK_REQUIRE(workspace_elems >= need && (need == 0 || workspace != nullptr),
             ZK_EWORKSPACE, "%s: workspace %lld < %lld floats", who,
             (long long)workspace_elems, (long long)need);
  const int64_t parts = rows == 0 ? 0 : need / hidden;
  if (rows == 0) {
    // nothing to differentiate; the reduce below writes dw = 0 (or keeps it)
  } else if (vec_ok(hidden, act_dtype, w_dtype, {dy, h, w, dres, dx, workspace})) {
    if (act_dtype == ZK_BF16) dispatch_w_bwd<bf16>(w_dtype, dy, h, w, rstd, dres, dx, workspace, parts, rows, hidden, s);
    else if (act_dtype == ZK_F16) dispatch_w_bwd<f16>(w_dtype, dy, h, w, rstd, dres, dx, workspace, parts, rows, hidden, s);
    else dispatch_w_bwd<float>(w_dtype, dy, h, w, rstd, dres, dx, workspace, parts, rows, hidden, s);
  } else {
    hipLaunchKernelGGL(rmsnorm_bwd_scalar, dim3(parts), dim3(256), 0, s, dy, h,
                       w, rstd, dres, dx, workspace, rows, hidden, act_dtype,
                       w_dtype);
  }
  hipLaunchKernelGGL(rmsnorm_dw_reduce, dim3((hidden + 63) / 64), dim3(1024),
                     0, s, workspace, parts, hidden, dw, w_dtype, accumulate);
  return launch_status(who);
}

static int check_bwd_args(const char* who, const void* dy, const void* h, const void* w,
                          const float* rstd, const void* dx, const void* dw, int64_t rows,
                          int64_t hidden, int act_dtype, int w_dtype) {
  ZK_REQUIRE(valid_dtype(act_dtype) && valid_dtype(w_dtype), ZK_EDTYPE,
             "%s: bad dtype code (%d, %d)", who, act_dtype, w_dtype);
  ZK_REQUIRE(rows >= 0 && hidden > 0, ZK_EINVAL, "%s: bad shape rows=%lld hidden=%lld", who,
             (long long)rows, (long long)hidden);
  ZK_REQUIRE(dy && h && w && rstd && dx && dw, ZK_EINVAL, "%s: null pointer", who);
  return ZK_OK;
}

// ---- the allocation-free variant's scratch ---------------------------------
// The dw partial rows of zk_rmsnorm_bwd_noalloc live in this file-scope device
// array: every GPU the library runs on holds its own copy (16 MiB) until the
// process ends.  Host code never passes the array's name to a kernel (on the
// host it is a stand-in, not a device address): the device address comes
// from hipGetSymbolAddress, looked up once per device with that device
// current, and that pointer is what the kernels receive.
static __device__ __align__(256) float scratch[ZK_RMSNORM_BWD_SCRATCH_FLOATS];

static constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static float* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of the current device's scratch array.
static int scratch_for_current_device(const char* who, float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  ZK_REQUIRE(e == hipSuccess, static_cast<int>(e), "%s: hipGetDevice failed: %s", who,
             hipGetErrorString(e));
  ZK_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, ZK_EUNSUPPORTED,
             "%s: device %d beyond the %d the scratch table holds", who, dev,
             kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    ZK_REQUIRE(e == hipSuccess && p != nullptr, e == hipSuccess ? ZK_EINVAL : static_cast<int>(e),
               "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, dev,
               hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return ZK_OK;
}

}  // namespace zk

extern "C" int zk_rmsnorm_bwd(const void* dy, const void* h, const void* w,
                              const float* rstd, const void* dres, void* dx,
                              void* dw, int accumulate, float* workspace,
                              int64_t workspace_elems, int64_t rows,
                              int64_t hidden, int act_dtype, int w_dtype,
                              zk_stream_t stream) {
  const int rc = check_bwd_args("zk_rmsnorm_bwd", dy, h, w, rstd, dx, dw, rows, hidden,
                                act_dtype, w_dtype);
  if (rc != ZK_OK) return rc;
  return rmsnorm_bwd_impl("zk_rmsnorm_bwd", dy, h, w, rstd, dres, dx, dw, accumulate,
                          workspace, workspace_elems, rows, hidden, act_dtype, w_dtype,
                          as_stream(stream));
}

extern "C" int zk_rmsnorm_bwd_noalloc(const void* dy, const void* h, const void* w,
                                      const float* rstd, const void* dres, void* dx,
                                      void* dw, int accumulate, int64_t rows,
                                      int64_t hidden, int act_dtype, int w_dtype,
                                      zk_stream_t stream) {
  const char* who = "zk_rmsnorm_bwd_noalloc";
  int rc = check_bwd_args(who, dy, h, w, rstd, dx, dw, rows, hidden, act_dtype, w_dtype);
  if (rc != ZK_OK) return rc;
  const int64_t need = zk_rmsnorm_bwd_workspace(rows, hidden);
  ZK_REQUIRE(need <= ZK_RMSNORM_BWD_SCRATCH_FLOATS, ZK_EWORKSPACE,
             "%s: rows=%lld hidden=%lld need %lld floats of scratch, more than the static "
             "%lld (ZK_RMSNORM_BWD_SCRATCH_FLOATS); use zk_rmsnorm_bwd with a workspace",
             who, (long long)rows, (long long)hidden, (long long)need,
             (long long)ZK_RMSNORM_BWD_SCRATCH_FLOATS);
  float* ws = nullptr;
  rc = scratch_for_current_device(who, &ws);
  if (rc != ZK_OK) return rc;
  return rmsnorm_bwd_impl(who, dy, h, w, rstd, dres, dx, dw, accumulate, ws,
                          ZK_RMSNORM_BWD_SCRATCH_FLOATS, rows, hidden, act_dtype, w_dtype,
                          as_stream(stream));
}
