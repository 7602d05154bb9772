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
  float* delta;   // backward workspace: fp32 [B, Hq, Sq]
  float* lse2;    // backward workspace: lse * log2(e), fp32 [B, Hq, Sq]
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
  // backward only, optional: the transpose of the RoPE rotation the forward
  // applied to Q and K, applied to dQ and dK before they are stored.  fp32
  // tables [rope_npos, d/2] (cos, sin), positions int64 [S] or null for
  // 0 .. S-1; rope_cos == null: no rotation.
  const float* rope_cos;
  const float* rope_sin;
  const int64_t* rope_pos;
  int64_t rope_npos;
  int rope_interleaved;
  // optional: the forward's O, the backward's dQ / dK / dV also stored
  // transposed, [H d, B S] (feature rows of t_ld elements, token b S + s along
  // a row), the layout the projections' weight gradients read; null: not stored
  void* o_t;
  void* dq_t;
  void* dk_t;
  void* dv_t;
  int64_t t_ld;
};

// Transposed store of a workgroup's rows (of O or a gradient): lane l of wave w holds
// x[nt][j] = element 32 nt + 8 (j / 4) + 4 g + j % 4 (g = l / 32) of row
// 32 w + l % 32 (the MFMA accumulator layout), NCOL = 32 x (waves) rows in
// all; they go out as the columns 0 .. ncols - 1 (ncols a multiple of 8) of
// the D feature rows at dst (row stride ld elements), scaled by `scale`.  The
// values pass through an LDS tile [D][NCOL] held by up to four arrays the
// caller no longer needs, RP feature rows each (p0 first); every wave must be
// done with them on entry.  16-byte stores, NCOL / 8 lanes per feature row.
// Ends with a barrier, so the arrays may be reused at once.
template <typename T, int D, int NCOL, int RP>
__device__ __forceinline__ void store_rows_transposed(const f32x16 (&x)[D / 32], float scale,
                                                      T* p0, T* p1, T* p2, T* p3, T* dst,
                                                      int64_t ld, int ncols) {
  static_assert(RP % 32 == 0 && D <= 4 * RP, "feature rows per array");
  constexpr int NT = 2 * NCOL;  // threads: 64 per 32 columns
  const int tid = threadIdx.x, l32 = tid & 31, g = (tid >> 5) & 1, wave = tid >> 6;
  const int c = 32 * wave + l32;
  auto row_ptr = [&](int r) __attribute__((always_inline)) {
    T* p = r < RP ? p0 : r < 2 * RP ? p1 : r < 3 * RP ? p2 : p3;
    return p + (r % RP) * NCOL;
  };
#pragma unroll
  for (int nt = 0; nt < D / 32; ++nt)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int r = 32 * nt + 8 * (j >> 2) + 4 * g + (j & 3);
      row_ptr(r)[c] = static_cast<T>(x[nt][j] * scale);
    }
  __syncthreads();
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  constexpr int CPR = NCOL / 8;  // 16-byte chunks per feature row
#pragma unroll
  for (int i = 0; i < D * CPR / NT; ++i) {
    const int id = NT * i + tid;
    const int r = id / CPR, col = 8 * (id % CPR);
    if (col < ncols)
      *reinterpret_cast<u32x4*>(dst + r * ld + col) = *reinterpret_cast<const u32x4*>(row_ptr(r) + col);
  }
  __syncthreads();
}

// MFMA selection by storage type: 32x32x16 (and 16x16x32) with fp32 accumulation.
template <typename T>
struct Mfma;

template <>
struct Mfma<bf16> {
  typedef bf16x8 vec8;
  static __device__ __forceinline__ f32x16 mma(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<f16> {
  typedef f16x8 vec8;
  static __device__ __forceinline__ f32x16 mma(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Transpose of the RoPE rotation, in registers.  x[nt][j] holds element
// d = 32 nt + 8 (j / 4) + 4 g + j % 4 of one row at sequence position `row`
// (the MFMA accumulator layout of a lane whose half is g), already in fp32.
// Half-split pairing (models/llama_simple.py:27-58): pairs (i, i + D / 2),
// i.e. nt and nt + D / 64 with the same j; interleaved pairing
// (models/llama_v2.py:151-177): pairs (2i, 2i + 1), i.e. j and j + 1 for
// even j.  With c, s the table values of pair i at the row's position, the
// forward rotated (a, b) -> (a c - b s, a s + b c); this applies
// (a, b) -> (a c + b s, b c - a s).
template <int D>
__device__ __forceinline__ void rope_inverse_regs(f32x16 (&x)[D / 32], const AttnArgs& a,
                                                  int64_t row, int g) {
  int64_t pos = a.rope_pos != nullptr ? a.rope_pos[row] : row;
  if (pos < 0) pos = 0;
  if (pos > a.rope_npos - 1) pos = a.rope_npos - 1;
  const float* ct = a.rope_cos + pos * (D / 2);
  const float* st = a.rope_sin + pos * (D / 2);
  if (a.rope_interleaved) {
#pragma unroll
    for (int nt = 0; nt < D / 32; ++nt)
#pragma unroll
      for (int a4 = 0; a4 < 4; ++a4) {
        const int d0 = 32 * nt + 8 * a4 + 4 * g;  // even: pairs (d0, d0+1), (d0+2, d0+3)
        const float2 c2 = *reinterpret_cast<const float2*>(ct + d0 / 2);
        const float2 s2 = *reinterpret_cast<const float2*>(st + d0 / 2);
        const float cs[2] = {c2.x, c2.y}, sn[2] = {s2.x, s2.y};
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const float u = x[nt][4 * a4 + 2 * p], w = x[nt][4 * a4 + 2 * p + 1];
          x[nt][4 * a4 + 2 * p] = fmaf(u, cs[p], w * sn[p]);
          x[nt][4 * a4 + 2 * p + 1] = fmaf(w, cs[p], -u * sn[p]);
        }
      }
  } else {
    constexpr int HALF_NT = D / 64;
#pragma unroll
    for (int nt = 0; nt < HALF_NT; ++nt)
#pragma unroll
      for (int a4 = 0; a4 < 4; ++a4) {
        const int i0 = 32 * nt + 8 * a4 + 4 * g;  // 4 consecutive pair indices
        const float4 c4 = *reinterpret_cast<const float4*>(ct + i0);
        const float4 s4 = *reinterpret_cast<const float4*>(st + i0);
        const float cs[4] = {c4.x, c4.y, c4.z, c4.w}, sn[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float u = x[nt][4 * a4 + e], w = x[nt + HALF_NT][4 * a4 + e];
          x[nt][4 * a4 + e] = fmaf(u, cs[e], w * sn[e]);
          x[nt + HALF_NT][4 * a4 + e] = fmaf(w, cs[e], -u * sn[e]);
        }
      }
  }
}

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

namespace zk {

// ---------------------------------------------------------------------------
// LDS tiles of D-element rows (D = 64 or 128, 2-byte elements), unpadded,
// with the 16-byte chunks of row r XOR-swizzled by sw(r) so that both access
// patterns the kernels use are free of bank conflicts:
//  * row reads (ds_read_b128): 16 lanes read one logical chunk of 16
//    consecutive rows -- sw(r) is a bijection on each run of 16 rows (per
//    row parity for D = 64, where two rows share a 256-byte bank row);
//  * transposed reads (ds_read_tr16_b64): a 32-lane half reads 4 consecutive
//    chunks of 4 consecutive rows -- sw maps those 4 rows to 4 disjoint
//    4-chunk groups.
template <int D>
__device__ __forceinline__ int tile_sw(int r) {
  if (D == 128) return ((r & 3) << 2) | ((r >> 2) & 3);
  return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
}
// Element offset of (row, col) in a swizzled tile; col % 8 is kept.
template <int D>
__device__ __forceinline__ int tile_off(int r, int col) {
  return r * D + ((((col >> 3) ^ tile_sw<D>(r))) << 3) + (col & 7);
}

// ---------------------------------------------------------------------------
// Transposed MFMA operand from a row-major swizzled LDS tile (gfx950
// ds_read_tr16_b64).
//
// The tile X holds X[r][c] at tile_off<D>(r, c).  The 32x32x16 MFMA A operand
// wants, in lane l, the 8 elements X^T[i][k] = X[k][i] with i = col0 + l % 32
// and k = klo + 0..3 (first half), k = khi + 0..3 (second half), where klo /
// khi may differ between the lane halves l < 32 and l >= 32.
// ds_read_tr16_b64 delivers, to lane i of a 16-lane group, element (i & 3) of
// the 8-byte chunks addressed by lanes (i >> 2) + 4e of that group
// (e = 0..3), so lane q of group G supplies the address of
// X[k0 + (q >> 2)][col0 + 16 (G & 1) + 4 (q & 3)].  The same layout serves a
// B operand whose columns are X's columns.
template <typename T, int D>
__device__ __forceinline__ typename Mfma<T>::vec8 lds_tr_operand(const T* tile, int col0,
                                                                 int klo, int khi) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const int lane = threadIdx.x & 63;
  const int q = lane & 15, G = lane >> 4;
  const int col = col0 + 16 * (G & 1) + 4 * (q & 3);
  const T* p0 = tile + tile_off<D>(klo + (q >> 2), col);
  const T* p1 = tile + tile_off<D>(khi + (q >> 2), col);
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p1));
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 w = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  return __builtin_bit_cast(typename Mfma<T>::vec8, w);
}

// ---------------------------------------------------------------------------
// Asynchronous tile loads: global memory -> LDS without staging registers
// (gfx950 buffer_load_dwordx4 ... lds).  One wave instruction writes 64
// consecutive 16-byte LDS chunks (LDS address = wave-uniform base + 16 lane);
// each lane picks the global chunk that belongs at its LDS position, which is
// how the XOR swizzle of tile_off is applied.  Rows at or past `nrows` are
// clamped to the last row so that every lane reads valid, finite data (the
// kernels mask those rows).  Completion is tracked by the wave's vmcnt.
//
// The loads use the buffer form (a resource over a wave-uniform base plus a
// 32-bit per-lane offset), not global_load_lds: the compiler's wait insertion
// counts a pending global-form LDS load as a second kind of LDS-counter event
// and then waits for every outstanding LDS read (lgkmcnt(0)) before the first
// use of any of them; with the buffer form it waits only for the read needed.
typedef __attribute__((address_space(1))) void gmem_void;
typedef __attribute__((address_space(3))) void lds_void;

// Raw (stride 0) buffer resource over [base, base + 2 GiB); offsets at or past
// the end read zeros instead of faulting.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}

// N bytes (4 or 16) per lane from base + voff + soff into LDS at dst + N lane.
template <int N>
__device__ __forceinline__ void dma_lds(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                        const void* dst) {
  static_assert(N == 4 || N == 16, "4 or 16 bytes per lane");
  if constexpr (N == 4)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)dst, 4, voff, soff, 0, 0);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)dst, 16, voff, soff, 0, 0);
}

template <typename T, int D, int ROWS, int NT = 256>
__device__ __forceinline__ void tile_load_async(T* tile, const T* gbase, int64_t ld,
                                                int64_t g0, int64_t nrows) {
  constexpr int CH = ROWS * D / 8;
  static_assert(CH % NT == 0, "tile must be a multiple of NT chunks");
  const int tid = threadIdx.x;
  // wave-uniform, so the LDS destination is computed in scalar registers
  const int wave_chunk0 = __builtin_amdgcn_readfirstlane(tid & ~63);
  // offsets from the tile's first row (< ROWS rows, so 32 bits suffice)
  const __amdgpu_buffer_rsrc_t r = raw_rsrc(gbase + g0 * ld);
#pragma unroll
  for (int i = 0; i < CH / NT; ++i) {
    const int p = i * NT + tid;
    const int row = p / (D / 8);
    const int c = (p % (D / 8)) ^ tile_sw<D>(row);
    int64_t gr = g0 + row;
    if (gr > nrows - 1) gr = nrows - 1;
    const uint32_t off = static_cast<uint32_t>(((gr - g0) * ld + c * 8) * static_cast<int64_t>(sizeof(T)));
    dma_lds<16>(r, off, 0, tile + (i * NT + wave_chunk0) * 8);
  }
}

// The same tile load with the per-lane address work done once.  For a tile
// of ROWS x D elements each of the NT threads moves NI = ROWS * D / (8 NT)
// chunks; chunk i of thread t lands in row RSTEP * i + t / (D / 8) at chunk
// position (t % (D / 8)) ^ sw(row), and since RSTEP is a multiple of 16 the
// swizzle (a function of row % 16) is the same for every i.  The per-lane
// byte offset inside the tile is therefore one 32-bit value, and each
// instruction's address is a wave-uniform base and row offset (scalar
// registers) plus that offset.  Tiles that run past `nrows` take the clamped path.
template <typename T, int D, int ROWS, int NT = 256>
struct TileLoader {
  static constexpr int NI = ROWS * D / 8 / NT;
  static constexpr int RSTEP = NT / (D / 8);
  static_assert(NI >= 1 && RSTEP % 16 == 0, "unsupported tile shape");
  uint32_t lane_off;  // bytes from the tile's first row

  __device__ __forceinline__ void init(int64_t ld) {
    const int tid = threadIdx.x;
    const int row = tid / (D / 8);
    const int c = (tid % (D / 8)) ^ tile_sw<D>(row);
    lane_off = static_cast<uint32_t>(row * ld * static_cast<int64_t>(sizeof(T)) + c * 16);
  }

  // Rows g0 .. g0 + ROWS - 1 must all lie below the tensor's row count.
  __device__ __forceinline__ void issue_full(T* tile, const T* gbase, int64_t ld,
                                             int64_t g0) const {
    const int wave_chunk0 = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) & ~63);
    const __amdgpu_buffer_rsrc_t r = raw_rsrc(gbase + g0 * ld);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const uint32_t soff =
          static_cast<uint32_t>(static_cast<int64_t>(i) * RSTEP * ld * static_cast<int64_t>(sizeof(T)));
      dma_lds<16>(r, lane_off, soff, tile + (i * NT + wave_chunk0) * 8);
    }
  }

  // `full` (wave-uniform) says that the tile lies below `nrows`; otherwise
  // rows past the end are clamped.
  __device__ __forceinline__ void issue(T* tile, const T* gbase, int64_t ld, int64_t g0,
                                        int64_t nrows, bool full) const {
    if (full)
      issue_full(tile, gbase, ld, g0);
    else
      tile_load_async<T, D, ROWS, NT>(tile, gbase, ld, g0, nrows);
  }
};

// Number of vector-memory instructions tile_load_async issues per wave.
template <int D, int ROWS>
constexpr int tile_load_insts() { return ROWS * D / 8 / 256; }

// s_waitcnt vmcnt(N) (expcnt / lgkmcnt left unconstrained), gfx9 encoding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Value of lane l ^ 32 (the other half of the wave) via gfx950's
// v_permlane32_swap: a VALU exchange, no LDS round trip.  swap(x, x) leaves
// {x[0..31], x[0..31]} in the first result and {x[32..63], x[32..63]} in
// the second, so lane l's partner value is the result from the other half.
__device__ __forceinline__ float other_half(float x) {
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                   false, false);
  return __uint_as_float((threadIdx.x & 32) ? sw[0] : sw[1]);
}

// True when key kj is visible from query qi (32-bit positions).
__device__ __forceinline__ bool visible32(int qi, int kj, int Sq, int Skv, int causal,
                                          int window) {
  return qi < Sq && kj < Skv && (!causal || kj <= qi) && (window <= 0 || kj > qi - window);
}

}  // namespace zk
