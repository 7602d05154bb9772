// 8-element vector load/store between storage types and fp32 registers.
#pragma once
#include "zk_common.h"

namespace zk {

template <typename T>
struct Vec8;

template <>
struct Vec8<float> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[8]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
};

template <>
struct Vec8<bf16> {
  static __device__ __forceinline__ void load(const bf16* p, float (&v)[8]) {
    const bf16x8 a = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = static_cast<float>(a[i]);
  }
  static __device__ __forceinline__ void store(bf16* p, const float (&v)[8]) {
    bf16x8 a;
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = static_cast<bf16>(v[i]);
    *reinterpret_cast<bf16x8*>(p) = a;
  }
};

template <>
struct Vec8<f16> {
  static __device__ __forceinline__ void load(const f16* p, float (&v)[8]) {
    const f16x8 a = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = static_cast<float>(a[i]);
  }
  static __device__ __forceinline__ void store(f16* p, const float (&v)[8]) {
    f16x8 a;
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = static_cast<f16>(v[i]);
    *reinterpret_cast<f16x8*>(p) = a;
  }
};

// 8 elements kept in their storage format (4 VGPRs for 2-byte types) and
// widened on use: lets a kernel keep several rows in flight cheaply.
template <typename T>
struct Raw8 {
  uint4 u;
  __device__ __forceinline__ void load(const T* p) { u = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ float operator[](int i) const {
    typedef T T8 __attribute__((ext_vector_type(8)));
    return static_cast<float>(__builtin_bit_cast(T8, u)[i]);
  }
  __device__ __forceinline__ void zero() { u = make_uint4(0, 0, 0, 0); }
  // Hide the value from the optimizer so widened copies are not kept alive
  // across a barrier (they are recomputed from the packed form instead).
  __device__ __forceinline__ void opaque() {
    asm volatile("" : "+v"(u.x), "+v"(u.y), "+v"(u.z), "+v"(u.w));
  }
};
template <>
struct Raw8<float> {
  float4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = reinterpret_cast<const float4*>(p)[0];
    b = reinterpret_cast<const float4*>(p)[1];
  }
  __device__ __forceinline__ float operator[](int i) const {
    const float4& v = i < 4 ? a : b;
    const int j = i & 3;
    return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
  }
  __device__ __forceinline__ void zero() { a = b = make_float4(0.f, 0.f, 0.f, 0.f); }
  __device__ __forceinline__ void opaque() {
    asm volatile("" : "+v"(a.x), "+v"(a.y), "+v"(a.z), "+v"(a.w));
    asm volatile("" : "+v"(b.x), "+v"(b.y), "+v"(b.z), "+v"(b.w));
  }
};

}  // namespace zk
