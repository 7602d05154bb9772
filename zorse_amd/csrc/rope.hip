// Rotary position embedding, applied in place to Q and K.
//
// One thread rotates 4 pairs of one (batch, position, head) row: for the
// half-split pairing it reads elements i..i+3 and i+d/2..i+d/2+3, for the
// interleaved pairing the 8 consecutive elements 2i..2i+7.  cos/sin come
// from fp32 tables [n_pos, d/2] built by the caller with the reference's
// own formula, so the kernel only does the rotation arithmetic (rotate_pair,
// rope_math.h).
#include "rope_math.h"

namespace zk {

template <typename T, int kPairing, bool kInverse>
__global__ __launch_bounds__(256) void rope_kernel(
    T* __restrict__ q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
    T* __restrict__ k, int64_t k_sb, int64_t k_ss, int64_t k_sh, int64_t B,
    int64_t S, int64_t Hq, int64_t Hkv, int64_t d,
    const float* __restrict__ cosT, const float* __restrict__ sinT,
    int64_t n_pos, const int64_t* __restrict__ positions) {
  const int64_t half = d / 2;
  const int64_t nq = (half + 3) / 4;  // quads of pairs per row
  const int64_t H = Hq + (k != nullptr ? Hkv : 0);
  const int64_t total = B * S * H * nq;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       t < total; t += stride) {
    int64_t r = t;
    const int64_t quad = r % nq; r /= nq;
    const int64_t h = r % H; r /= H;
    const int64_t s = r % S;
    const int64_t b = r / S;
    T* row = h < Hq ? q + b * q_sb + s * q_ss + h * q_sh
                    : k + b * k_sb + s * k_ss + (h - Hq) * k_sh;
    int64_t pos = positions != nullptr ? positions[s] : s;
    if (pos < 0) pos = 0;
    if (pos >= n_pos) pos = n_pos - 1;
    const float* crow = cosT + pos * half;
    const float* srow = sinT + pos * half;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t i = quad * 4 + j;
      if (i < half) {
        const int64_t i1 = kPairing == ZK_ROPE_HALF ? i : 2 * i;
        const int64_t i2 = kPairing == ZK_ROPE_HALF ? i + half : 2 * i + 1;
        float y1, y2;
        rotate_pair<T, kPairing, kInverse>(to_f32(row[i1]), to_f32(row[i2]),
                                           crow[i], srow[i], y1, y2);
        row[i1] = from_f32<T>(y1);
        row[i2] = from_f32<T>(y2);
      }
    }
  }
}

// Vectorised path for head_dim 64 / 128 with 16-byte aligned rows: a thread
// rotates 8 pairs with 16-byte accesses; the grid is (position blocks,
// heads, batch), so no index arithmetic divides.
// One thread's 8 pairs of one (position, head) row, 16-byte accesses.
template <typename T, int D, int kPairing, bool kInverse>
__device__ __forceinline__ void rope_chunk8(T* row, int i0, const float (&c)[8],
                                            const float (&sn)[8]) {
  constexpr int HALF = D / 2;
  float x1[8], x2[8], y1[8], y2[8];
  if (kPairing == ZK_ROPE_HALF) {
    Vec8<T>::load(row + i0, x1);
    Vec8<T>::load(row + i0 + HALF, x2);
  } else {
    float a[8], bb[8];
    Vec8<T>::load(row + 2 * i0, a);
    Vec8<T>::load(row + 2 * i0 + 8, bb);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x1[j] = a[2 * j];
      x2[j] = a[2 * j + 1];
      x1[j + 4] = bb[2 * j];
      x2[j + 4] = bb[2 * j + 1];
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) rotate_pair<T, kPairing, kInverse>(x1[j], x2[j], c[j], sn[j], y1[j], y2[j]);
  if (kPairing == ZK_ROPE_HALF) {
    Vec8<T>::store(row + i0, y1);
    Vec8<T>::store(row + i0 + HALF, y2);
  } else {
    float a[8], bb[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a[2 * j] = y1[j];
      a[2 * j + 1] = y2[j];
      bb[2 * j] = y1[j + 4];
      bb[2 * j + 1] = y2[j + 4];
    }
    Vec8<T>::store(row + 2 * i0, a);
    Vec8<T>::store(row + 2 * i0 + 8, bb);
  }
}

// Vectorised path for head_dim 64 / 128 with 16-byte aligned rows and few
// heads: a thread rotates 8 pairs of one row; the grid is (position blocks,
// heads, batch), so no index arithmetic divides.
template <typename T, int D, int kPairing, bool kInverse>
__global__ __launch_bounds__(256) void rope_vec_kernel(
    T* __restrict__ q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
    T* __restrict__ k, int64_t k_sb, int64_t k_ss, int64_t k_sh, int64_t S, int64_t Hq,
    const float* __restrict__ cosT, const float* __restrict__ sinT, int64_t n_pos,
    const int64_t* __restrict__ positions) {
  constexpr int HALF = D / 2;
  constexpr int TPR = HALF / 8;        // threads per (position, head) row
  constexpr int RPB = 256 / TPR;       // positions per workgroup
  const int64_t s = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / TPR;
  if (s >= S) return;
  const int64_t h = blockIdx.y, b = blockIdx.z;
  const int i0 = (threadIdx.x % TPR) * 8;  // first pair of this thread
  T* row = h < Hq ? q + b * q_sb + s * q_ss + h * q_sh
                  : k + b * k_sb + s * k_ss + (h - Hq) * k_sh;
  int64_t pos = positions != nullptr ? positions[s] : s;
  if (pos < 0) pos = 0;
  if (pos >= n_pos) pos = n_pos - 1;
  float c[8], sn[8];
  Vec8<float>::load(cosT + pos * HALF + i0, c);
  Vec8<float>::load(sinT + pos * HALF + i0, sn);
  rope_chunk8<T, D, kPairing, kInverse>(row, i0, c, sn);
}

// Position-major path for many heads: a workgroup rotates every q and k head
// of one (batch, position) -- with heads contiguous in memory, one run of
// (Hq + Hkv) d elements -- and each thread reads its cos / sin values once
// (256 threads and HALF / 8 chunks per row: a thread's pair offset is the
// same in every head it visits).
template <typename T, int D, int kPairing, bool kInverse>
__global__ __launch_bounds__(256) void rope_pos_kernel(
    T* __restrict__ q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
    T* __restrict__ k, int64_t k_sb, int64_t k_ss, int64_t k_sh, int64_t Hq, int64_t H,
    const float* __restrict__ cosT, const float* __restrict__ sinT, int64_t n_pos,
    const int64_t* __restrict__ positions) {
  constexpr int HALF = D / 2;
  constexpr int CPH = HALF / 8;  // 8-pair chunks per head row
  static_assert(256 % CPH == 0, "chunk offset must be fixed per thread");
  const int64_t s = blockIdx.x, b = blockIdx.y;
  const int i0 = (threadIdx.x % CPH) * 8;
  int64_t pos = positions != nullptr ? positions[s] : s;
  if (pos < 0) pos = 0;
  if (pos >= n_pos) pos = n_pos - 1;
  float c[8], sn[8];
  Vec8<float>::load(cosT + pos * HALF + i0, c);
  Vec8<float>::load(sinT + pos * HALF + i0, sn);
  T* qrow = q + b * q_sb + s * q_ss;
  T* krow = k != nullptr ? k + b * k_sb + s * k_ss : nullptr;
  for (int64_t h = threadIdx.x / CPH; h < H; h += 256 / CPH) {
    T* row = h < Hq ? qrow + h * q_sh : krow + (h - Hq) * k_sh;
    rope_chunk8<T, D, kPairing, kInverse>(row, i0, c, sn);
  }
}

template <typename T, int D>
static void launch_rope_vec(int pairing, int inverse, void* q, int64_t q_sb, int64_t q_ss,
                            int64_t q_sh, void* k, int64_t k_sb, int64_t k_ss, int64_t k_sh,
                            int64_t B, int64_t S, int64_t Hq, int64_t Hkv, const float* c,
                            const float* sn, int64_t n_pos, const int64_t* pos, hipStream_t st) {
  constexpr int RPB = 256 / (D / 16);
  const int64_t H = Hq + (k != nullptr ? Hkv : 0);
  // position-major once a position's rows fill half a workgroup's threads
  const bool by_pos = H * (D / 16) >= 128 && S < 0x7fffffff;
  const dim3 grid = by_pos ? dim3(static_cast<unsigned>(S), static_cast<unsigned>(B))
                           : dim3(static_cast<unsigned>((S + RPB - 1) / RPB),
                                  static_cast<unsigned>(H), static_cast<unsigned>(B));
#define ZK_ROPEV(P, I)                                                                       \
  do {                                                                                       \
    if (by_pos)                                                                              \
      hipLaunchKernelGGL((rope_pos_kernel<T, D, P, I>), grid, dim3(256), 0, st, (T*)q, q_sb,  \
                         q_ss, q_sh, (T*)k, k_sb, k_ss, k_sh, Hq, H, c, sn, n_pos, pos);     \
    else                                                                                     \
      hipLaunchKernelGGL((rope_vec_kernel<T, D, P, I>), grid, dim3(256), 0, st, (T*)q, q_sb,  \
                         q_ss, q_sh, (T*)k, k_sb, k_ss, k_sh, S, Hq, c, sn, n_pos, pos);     \
  } while (0)
  if (pairing == ZK_ROPE_HALF) {
    if (inverse) ZK_ROPEV(ZK_ROPE_HALF, true); else ZK_ROPEV(ZK_ROPE_HALF, false);
  } else {
    if (inverse) ZK_ROPEV(ZK_ROPE_INTERLEAVED, true); else ZK_ROPEV(ZK_ROPE_INTERLEAVED, false);
  }
#undef ZK_ROPEV
}

template <typename T>
static void launch_rope(int pairing, int inverse, void* q, int64_t q_sb,
                        int64_t q_ss, int64_t q_sh, void* k, int64_t k_sb,
                        int64_t k_ss, int64_t k_sh, int64_t B, int64_t S,
                        int64_t Hq, int64_t Hkv, int64_t d, const float* c,
                        const float* sn, int64_t n_pos, const int64_t* pos,
                        hipStream_t st) {
  const int64_t H = Hq + (k != nullptr ? Hkv : 0);
  const int64_t total = B * S * H * ((d / 2 + 3) / 4);
  int64_t grid = (total + 255) / 256;
  const int64_t cap = static_cast<int64_t>(device_cus()) * 16;
  if (grid > cap) grid = cap;
  if (grid < 1) grid = 1;
#define ZK_ROPE(P, I)                                                          \
  hipLaunchKernelGGL((rope_kernel<T, P, I>), dim3(grid), dim3(256), 0, st,     \
                     (T*)q, q_sb, q_ss, q_sh, (T*)k, k_sb, k_ss, k_sh, B, S, Hq, \
                     Hkv, d, c, sn, n_pos, pos)
  if (pairing == ZK_ROPE_HALF) {
    if (inverse) ZK_ROPE(ZK_ROPE_HALF, true); else ZK_ROPE(ZK_ROPE_HALF, false);
  } else {
    if (inverse) ZK_ROPE(ZK_ROPE_INTERLEAVED, true); else ZK_ROPE(ZK_ROPE_INTERLEAVED, false);
  }
#undef ZK_ROPE
}

}  // namespace zk

using namespace zk;

extern "C" int zk_rope(void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                       void* k, int64_t k_sb, int64_t k_ss, int64_t k_sh,
                       int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t d,
                       const float* cos, const float* sin, int64_t n_pos,
                       const int64_t* positions, int pairing, int inverse,
                       int dtype, zk_stream_t stream) {
  ZK_REQUIRE(valid_dtype(dtype), ZK_EDTYPE, "zk_rope: bad dtype %d", dtype);
  ZK_REQUIRE(pairing == ZK_ROPE_HALF || pairing == ZK_ROPE_INTERLEAVED,
             ZK_EINVAL, "zk_rope: bad pairing %d", pairing);
  ZK_REQUIRE(B >= 0 && S >= 0 && Hq >= 0 && Hkv >= 0 && d > 0 && d % 2 == 0,
             ZK_EINVAL, "zk_rope: bad shape (d must be even, got %lld)",
             (long long)d);
  ZK_REQUIRE(q && cos && sin, ZK_EINVAL, "zk_rope: null pointer");
  ZK_REQUIRE(positions != nullptr || n_pos >= S, ZK_EINVAL,
             "zk_rope: table has %lld positions < S=%lld", (long long)n_pos,
             (long long)S);
  ZK_REQUIRE(n_pos > 0, ZK_EINVAL, "zk_rope: empty table");
  if (B == 0 || S == 0 || Hq + Hkv == 0) return ZK_OK;
  hipStream_t st = as_stream(stream);
  // 16-byte vector path: 2-byte types, d 64 / 128, aligned rows and heads,
  // grid dimensions within range
  const int64_t H = Hq + (k != nullptr ? Hkv : 0);
  bool vec = dtype != ZK_F32 && (d == 64 || d == 128) && aligned(q, 16) &&
             (k == nullptr || aligned(k, 16)) && H < 65536 && B < 65536 &&
             S / (256 / (d / 16)) < 0x7fffffff;
  vec = vec && q_sb % 8 == 0 && q_ss % 8 == 0 && q_sh % 8 == 0;
  if (k != nullptr) vec = vec && k_sb % 8 == 0 && k_ss % 8 == 0 && k_sh % 8 == 0;
  if (vec) {
#define ZK_VEC(T, D) launch_rope_vec<T, D>(pairing, inverse, q, q_sb, q_ss, q_sh, k, k_sb, k_ss, k_sh, B, S, Hq, Hkv, cos, sin, n_pos, positions, st)
    if (dtype == ZK_BF16) {
      if (d == 128) ZK_VEC(bf16, 128); else ZK_VEC(bf16, 64);
    } else {
      if (d == 128) ZK_VEC(f16, 128); else ZK_VEC(f16, 64);
    }
#undef ZK_VEC
    return launch_status("zk_rope");
  }
  if (dtype == ZK_BF16)
    launch_rope<bf16>(pairing, inverse, q, q_sb, q_ss, q_sh, k, k_sb, k_ss, k_sh, B, S, Hq, Hkv, d, cos, sin, n_pos, positions, st);
  else if (dtype == ZK_F16)
    launch_rope<f16>(pairing, inverse, q, q_sb, q_ss, q_sh, k, k_sb, k_ss, k_sh, B, S, Hq, Hkv, d, cos, sin, n_pos, positions, st);
  else
    launch_rope<float>(pairing, inverse, q, q_sb, q_ss, q_sh, k, k_sb, k_ss, k_sh, B, S, Hq, Hkv, d, cos, sin, n_pos, positions, st);
  return launch_status("zk_rope");
}
