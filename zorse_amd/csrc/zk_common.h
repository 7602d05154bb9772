// Shared helpers for the gfx950 kernels of libzorse_amd.so: storage-type
// conversion, vector load/store types, error reporting across the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/zorse_amd.h"

namespace zk {

typedef __bf16 bf16;
typedef _Float16 f16;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---- error reporting (host) -------------------------------------------------
void set_error(const char* fmt, ...);
void clear_error();
int launch_status(const char* what);  // maps hipGetLastError() to a status

#define ZK_REQUIRE(cond, code, ...)  \
  do {                               \
    if (!(cond)) {                   \
      ::zk::set_error(__VA_ARGS__);  \
      return (code);                 \
    }                                \
  } while (0)

inline bool valid_dtype(int dt) {
  return dt == ZK_F32 || dt == ZK_F16 || dt == ZK_BF16;
}
inline int dtype_bytes(int dt) { return dt == ZK_F32 ? 4 : 2; }
inline bool aligned(const void* p, int bytes) {
  return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}
inline hipStream_t as_stream(zk_stream_t s) {
  return reinterpret_cast<hipStream_t>(s);
}

// ---- device conversions -----------------------------------------------------
// Storage types convert through float; float->bf16/f16 use the hardware
// round-to-nearest-even conversions (v_cvt_pk_bf16_f32 / v_cvt_f16_f32).
template <typename T>
__device__ __forceinline__ float to_f32(T v) {
  return static_cast<float>(v);
}
template <typename T>
__device__ __forceinline__ T from_f32(float v) {
  return static_cast<T>(v);
}
// Round a float to the storage precision of T and widen back.
template <typename T>
__device__ __forceinline__ float round_to(float v) {
  return static_cast<float>(static_cast<T>(v));
}
template <>
__device__ __forceinline__ float round_to<float>(float v) {
  return v;
}

// Generic element load/store by runtime dtype code (for the cold paths).
__device__ __forceinline__ float load_dt(const void* p, int64_t i, int dt) {
  if (dt == ZK_F32) return reinterpret_cast<const float*>(p)[i];
  if (dt == ZK_BF16) return to_f32(reinterpret_cast<const bf16*>(p)[i]);
  return to_f32(reinterpret_cast<const f16*>(p)[i]);
}
__device__ __forceinline__ void store_dt(void* p, int64_t i, int dt, float v) {
  if (dt == ZK_F32)
    reinterpret_cast<float*>(p)[i] = v;
  else if (dt == ZK_BF16)
    reinterpret_cast<bf16*>(p)[i] = from_f32<bf16>(v);
  else
    reinterpret_cast<f16*>(p)[i] = from_f32<f16>(v);
}

// ---- wavefront reductions (64 lanes) ---------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Number of CUs on the current device (cached per device).
int device_cus();

}  // namespace zk
