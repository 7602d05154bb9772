// Shared definitions for the attention kernels (forward and backward).
#pragma once
#include "zk_common.h"

namespace zk {

static constexpr float kLog2e = 1.4426950408889634f;

// Kernel-side view of zk_attn_desc plus the data pointers.
struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const float* lse;
  void* out;      // forward: O ; backward: unused
  float* lse_out; // forward: lse
  void* dq;
  void* dk;
  void* dv;
  float* dq_acc;  // backward workspace: fp32 [B, Sq, Hq, d]
  float* delta;   // backward workspace: fp32 [B, Hq, Sq]
  int64_t B, Sq, Skv, Hq, Hkv, d;
  int64_t q_sb, q_ss, q_sh;
  int64_t k_sb, k_ss, k_sh;
  int64_t v_sb, v_ss, v_sh;
  int64_t o_sb, o_ss, o_sh;
  int64_t dq_sb, dq_ss, dq_sh;
  int64_t dk_sb, dk_ss, dk_sh;
  int64_t dv_sb, dv_ss, dv_sh;
  float scale;
  float scale_log2;  // scale * log2(e)
  int causal;
  int64_t window;
};

// MFMA selection by storage type: 32x32x16 with fp32 accumulation.
template <typename T>
struct Mfma;

template <>
struct Mfma<bf16> {
  typedef bf16x8 vec8;
  static __device__ __forceinline__ f32x16 mma(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<f16> {
  typedef f16x8 vec8;
  static __device__ __forceinline__ f32x16 mma(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// True when key `kj` is visible from query `qi`.
__device__ __forceinline__ bool attn_visible(int64_t qi, int64_t kj,
                                             int64_t Skv, int causal,
                                             int64_t window) {
  if (kj >= Skv) return false;
  if (causal && kj > qi) return false;
  if (window > 0 && kj <= qi - window) return false;
  return true;
}

}  // namespace zk
