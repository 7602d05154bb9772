// The rotary-embedding rotation of one pair, shared by the RoPE pass
// (rope.hip) and the q|k|v GEMM's RoPE epilogue (gemm_kernels.h), so that the
// two round identically:
//   half-split (HF rotate_half, per-op rounding in the storage type):
//     y1 = r(r(x1 c) + r(-x2 s))      y2 = r(r(x2 c) + r(x1 s))
//   interleaved (complex product in fp32, one rounding by the caller's store):
//     y1 = x1 c - x2 s                y2 = x1 s + x2 c
//     (each as one fma of the first product and the other, rounded, product)
// The inverse (backward) applies the transpose rotation with the same
// rounding structure as autograd of those expressions.
#pragma once
#include "vec.h"

namespace zk {

template <typename T, int kPairing, bool kInverse>
__device__ __forceinline__ void rotate_pair(float x1, float x2, float c,
                                            float s, float& y1, float& y2) {
  if (kPairing == ZK_ROPE_HALF) {
    if (!kInverse) {
      y1 = round_to<T>(round_to<T>(x1 * c) + round_to<T>(-x2 * s));
      y2 = round_to<T>(round_to<T>(x2 * c) + round_to<T>(x1 * s));
    } else {
      // d/dx of the forward: dx1 = dy1 c + dy2 s, dx2 = dy2 c - dy1 s
      y1 = round_to<T>(round_to<T>(x1 * c) + round_to<T>(x2 * s));
      y2 = round_to<T>(round_to<T>(x2 * c) - round_to<T>(x1 * s));
    }
  } else {
    // written as explicit fmas so that every kernel using this rotation
    // rounds the same (left to the compiler, a * b - c * d contracts
    // differently from one kernel to another)
    if (!kInverse) {
      y1 = fmaf(x1, c, -(x2 * s));
      y2 = fmaf(x1, s, x2 * c);
    } else {
      y1 = fmaf(x1, c, x2 * s);
      y2 = fmaf(x2, c, -(x1 * s));
    }
  }
}

}  // namespace zk
