// Projection GEMMs for gfx950 (bf16 / fp16 storage, fp32 accumulation):
//
//   C[M, N] = op(A) op(B)^T (+ R[M, N])
//
// with each operand either contiguous along the reduction ("NT": A [M, K],
// B [N, K], the nn.Linear forward x W^T) or along its output dimension
// ("K-major": A [K, M], B [K, N]).  The layer's backward takes both forms
// from the tensors as the forward left them: the input gradient dY W reads
// dY [T, out] along the reduction and W [out, in] K-major; the weight
// gradient dY^T X reads dY [T, out] and X [T, in] both K-major.  No operand
// is ever transposed in memory.  One fp32 rounding of the accumulated sum
// (plus R) to the storage type.
//
// Workgroup = 4 waves, tile = 256 x 256, one workgroup per CU (160 KB LDS,
// one wave per SIMD).  Each wave owns a 128 x 128 block: 8 x 8 MFMA blocks of
// v_mfma_f32_16x16x32 whose 256 accumulators live in AGPRs, so the 256
// architectural VGPRs hold two sets of operands (one per 32-deep substep of a
// 64-deep K step), the next read during the current one's MFMAs.  (The same
// pipeline on 4 x 4 blocks of v_mfma_f32_32x32x16 ran 6-10 % slower at the
// 7B shapes.)
//
// Tiles reach LDS through buffer_load_dwordx4 ... lds (16 bytes per lane).
// An NT operand tile is 256 rows x 64 k (128-byte row segments, chunks
// XOR-swizzled by nt_sw) read by ds_read_b128; a K-major operand tile is
// 64 k-rows x 256 columns (512-byte row segments, swizzled by kmaj_sw) read
// by ds_read_b64_tr_b16, which hands each lane 4 consecutive k of one column
// -- two of them make the MFMA operand the b128 read gives an NT tile.  A
// sits in a ring of three stages and B in a ring of two, so A's loads run
// two K steps ahead and B's one; the refill of each K step is spread one
// load per eight MFMAs over the whole step, because a burst of loads fills
// the texture unit's command queue and stalls the issuing wave (counters:
// SQ_VMEM_TA_CMD_FIFO_FULL), and the operand reads likewise go two per eight
// MFMAs (SQ_LDS_CMD_FIFO_FULL).  The loads are issued from inline assembly:
// with an LDS DMA visible to it, the compiler's wait insertion waits for
// every load in flight before any LDS read; the kernel orders them itself
// with exact vmcnt waits (loads complete in issue order) and one barrier per
// K step.
//
// Workgroups are remapped so that the 32 CUs of one XCD (dispatch order
// round-robins XCDs) take consecutive tiles, ordered in groups of four M
// tiles, so each XCD's L2 serves a 4 x 8 block of tiles.
//
// Shapes off that grid, fp32 operands, and leading dimensions past the
// buffer-resource range go to gemm_gen_kernel: 128 x 128 tiles staged
// through registers with masked loads and stores (any M, N, K).
//
// This header holds the kernels; gemm.hip launches the NT forms (the
// forward products and the SwiGLU-epilogue instance) and the general kernel,
// gemm_kmajor.hip the tiled forms with a K-major operand (the backward
// products).  The two are compiled apart because the K-major forms need
// another register-assignment order from the compiler: with its default the
// 256 accumulators of the both-K-major form were rotated between AGPRs by
// ~80 moves per loop pass (about 10 % of that product's time); with
// -greedy-reverse-local-assignment none are, while the NT forms do better
// with the default.
#pragma once
#include "attn_common.h"
#include "rope_math.h"
#include "vec.h"

namespace zk {
namespace gemm {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int GROUP_M = 4;  // 8 and 16 measured slower in the 7B stage

typedef int v4i __attribute__((ext_vector_type(4)));

// Raw buffer resource over [base, base + 2 GiB) as four scalar dwords.
__device__ __forceinline__ v4i rsrc_words(const void* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  v4i r;
  r[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu));
  r[1] = __builtin_amdgcn_readfirstlane(static_cast<int>((a >> 32) & 0xffffu));
  r[2] = 0x7fffffff;
  r[3] = 0x00020000;
  return r;
}

template <typename T>
__device__ __forceinline__ uint32_t lds_addr(const T* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const T*)(p)));
}

// 16 bytes per lane from r + voff + soff into LDS at lds + 16 lane.  The
// asm writes the LDS address into M0 and declares M0 clobbered, so the
// compiler keeps nothing of its own there across it.  (clang warns that M0
// is a reserved register -- the compiler sets it right before each of its
// own uses -- and that a reserved register may not be preserved across the
// asm, which is what the clobber says; binding the address to M0 as an
// input operand instead made the register allocator shuttle accumulators
// between AGPRs and VGPRs in the main loop.)
__device__ __forceinline__ void dma16(v4i r, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :: "v"(voff), "s"(r), "s"(soff), "s"(lds) : "memory", "m0");
}

// Operands and outputs of one launch.  EPI 0: c = a b^T (+ r); EPI 2: c =
// a b^T with the rotary embedding applied to its first rcols columns (the q
// and k heads of a q|k|v projection, heads of rhalf * 2 columns, row m the
// token at sequence position m % rS, position index rpos[m % rS] or m % rS
// into the fp32 tables rcos / rsin [rnpos, rhalf], pairing rpair), exactly as
// the RoPE pass would rotate the stored product; EPI 1 (the
// gate|up projection with the SwiGLU epilogue): b = W_gate, b2 = W_up (each
// [F, K]), N = 2F, c / c2 = g / u (row stride ldc), z = SwiGLU(g, u) and,
// when zt is not NULL, zt = z^T.
struct GemmArgs {
  const void* a;
  int64_t lda;
  const void* b;
  const void* b2;
  int64_t ldb;
  void* c;
  void* c2;
  int64_t ldc;
  const void* r;
  int64_t ldr;
  void* z;
  int64_t ldz;
  void* zt;
  int64_t ldzt;
  int64_t M, N, K;
  const float* rcos;
  const float* rsin;
  const int64_t* rpos;
  int64_t rnpos, rS, rcols;
  int rhalf, rpair;
};

// NT tile swizzle: the 16-byte chunk c of row r sits at chunk position
// c ^ nt_sw(r).  An operand read (ds_read_b128) gives lane l row r0 + l % 16,
// chunk l / 16 (XOR 4 in substep 1), and gfx950 serves a wave's b128 read in
// four passes of 16 lanes, {0-3, 12-15, 20-23, 24-27}, {4-7, 8-11, 16-19,
// 28-31} and the same plus 32 (measured: two lanes conflict iff they are in
// one pass).  Two 128-byte rows fill one 256-byte bank row, so a lane's bank
// group is 8 (r & 1) + (chunk ^ nt_sw(r)).  With m = (r / 2) % 8, nt_sw takes
// the rows of m in {0, 1, 6, 7} to {0 .. 3} and those of m in {2 .. 5} to
// {4 .. 7}; a pass pairs chunk c on the first set of rows with chunk c ^ 1 on
// the second, so its 16 lanes land on 16 different bank groups.  (The
// attention tiles' tile_sw<64> put two lanes of each pass on one bank group.)
__device__ __forceinline__ int nt_sw(int r) {
  const int m = (r >> 1) & 7;
  return ((((m >> 1) ^ (m >> 2)) & 1) << 2) | (((m >> 2) & 1) << 1) | (m & 1);
}
__device__ __forceinline__ int nt_off(int r, int col) {
  return r * BK + ((((col >> 3) ^ nt_sw(r))) << 3) + (col & 7);
}

// An NT tile: ROWS x 64 (128-byte rows, chunks swizzled by nt_sw) in eight
// instructions of 32 rows; instruction i of wave w fills LDS chunks
// 256 i + 64 w .. +63, lane l the chunk of row 32 i + (64 w + l) / 8.
template <typename T>
struct TileDma {
  static constexpr int D = BK, NT = 256, RSTEP = NT / (D / 8);
  uint32_t lane_off;   // bytes from the tile's first row
  uint32_t lane_off8;  // bytes from the wave's first row (8 rows per wave)
  int wave_el;         // wave-uniform
  __device__ __forceinline__ void init(int64_t ld) {
    const int tid = threadIdx.x;
    const int row = tid / (D / 8);
    const int c = (tid % (D / 8)) ^ nt_sw(row);
    lane_off = static_cast<uint32_t>(row * ld * static_cast<int64_t>(sizeof(T)) + c * 16);
    lane_off8 = static_cast<uint32_t>((row & 7) * ld * static_cast<int64_t>(sizeof(T)) + c * 16);
    wave_el = __builtin_amdgcn_readfirstlane(tid >> 6) * 64 * 8;
  }
  // piece i: this wave's 8 tile rows (32 i + 8 w ..) from the 8 source rows
  // at src + soff bytes (src wave-uniform)
  __device__ __forceinline__ void issue_wave_rows(T* tile, const T* src, uint32_t soff,
                                                  int i) const {
    dma16(rsrc_words(src), lane_off8, soff, lds_addr(tile + wave_el) + i * NT * 16);
  }
  // piece i (rows 32 i .. 32 i + 31) of the tile whose first row is `gbase`
  __device__ __forceinline__ void issue(T* tile, const T* gbase, int64_t ld, int i) const {
    const v4i r = rsrc_words(gbase);
    const uint32_t soff =
        static_cast<uint32_t>(static_cast<int64_t>(i) * RSTEP * ld * static_cast<int64_t>(sizeof(T)));
    dma16(r, lane_off, soff, lds_addr(tile + wave_el) + i * NT * 16);
  }
};

// A K-major tile: 64 k-rows x 256 columns (512-byte rows); the 16-byte chunk
// c of row k sits at chunk position c ^ kmaj_sw(k).  One transposed operand
// read of a 32-lane half touches the same 32-byte column pair of rows
// {k0 .. k0 + 3, k0 + 8 .. k0 + 11} (k0 a multiple of 4 with bit 2 clear, or
// k0 + 4 ..): kmaj_sw sends those eight rows to eight different 32-byte bank
// groups of the 256-byte bank row, so the read is free of bank conflicts.
__device__ __forceinline__ int kmaj_sw(int k) { return 2 * ((k & 3) | ((k >> 1) & 4)); }

// Loads of a K-major tile, eight instructions of two rows: instruction i of
// wave w fills rows 2 (w & 1) + 8 (w >> 1) + 4 (i & 1) + 16 (i >> 1) and the
// row after it (lanes 0-31, 32-63), so each lane's row keeps the same
// kmaj_sw in every instruction and its byte offset is one 32-bit value.
template <typename T>
struct TileDmaK {
  uint32_t lane_off;  // bytes from the tile's first row
  int wave_row;       // wave-uniform
  __device__ __forceinline__ void init(int64_t ld) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    wave_row = 2 * (w & 1) + 8 * (w >> 1);
    const int row = wave_row + (lane >> 5);
    const int c = (lane & 31) ^ kmaj_sw(row);
    lane_off = static_cast<uint32_t>(row * ld * static_cast<int64_t>(sizeof(T)) + c * 16);
  }
  // piece i of the tile whose first row (k) and column are at `gbase`
  __device__ __forceinline__ void issue(T* tile, const T* gbase, int64_t ld, int i) const {
    const int ri = 4 * (i & 1) + 16 * (i >> 1);
    const uint32_t soff = static_cast<uint32_t>(ri * ld * static_cast<int64_t>(sizeof(T)));
    dma16(rsrc_words(gbase), lane_off, soff, lds_addr(tile + (wave_row + ri) * 256));
  }
};

// Element offset, in a K-major tile, of this lane's first transposed read
// for the 16-column block at colw: row k = 8 (l / 16) + (l % 16) / 4, column
// colw + 4 (l % 4).  The read of column block colw + 16 r at substep s (k +
// 32 s) is at (base ^ 16 r) + 8192 s, and its second half (k + 4) 1024
// elements further: the XOR touches the chunk bits 1-3, where the base holds
// kmaj_sw; the base's k is below 32 with bit 2 clear, so the two steps are
// plain adds (immediate offsets of the read) and neither changes kmaj_sw.
__device__ __forceinline__ int kmaj_base(int colw) {
  const int lane = threadIdx.x & 63;
  const int k = 8 * (lane >> 4) + ((lane & 15) >> 2);
  const int col = colw + 4 * (lane & 3);
  return k * 256 + (((col >> 3) ^ kmaj_sw(k)) << 3) + (col & 7);
}

// The MFMA operand (lane l: 8 consecutive k from 8 (l / 16) of column
// l % 16 of the block) from a K-major tile: two ds_read_b64_tr_b16, each of
// which gives lane i of a 16-lane group element (i & 3) of the 8-byte runs
// addressed by lanes (i >> 2) + 4 e, e = 0..3 -- i.e. column i of rows
// k .. k + 3.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::vec8 kmaj_operand(const T* tile, int off) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + off));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + off + 1024));
  return __builtin_bit_cast(typename Mfma<T>::vec8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}

// silu(g) = g / (1 + e^-g) from the hardware exp2 and reciprocal (about one
// fp32 ulp each): the epilogue's four waves per CU evaluate it for every
// output element of the tile while the CU's MFMAs wait, so the IEEE exp and
// division (about four times the instructions) would cost ~10 % of the GEMM.
// Rounded to bf16 / fp16 right after, it differs from the IEEE form in about
// one element in 10^4, by one ulp of the storage type.
__device__ __forceinline__ float silu_fast(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504088896341f));
}

// AKM / BKM: operand A / B is K-major (see the top of the file).  EPI 1
// takes NT operands only.
// Products with A along the reduction whose 256 x 256 tiles would occupy at
// most half the CUs (e.g. a 4096 x 2048 product: 128 tiles on 256 CUs) run on
// 128 x 256 tiles instead, twice the workgroups with half the work each and
// every output summed in the same order.
inline bool half_tiles(int64_t nwg) { return nwg > 0 && 2 * nwg <= device_cus(); }

// Operand-read order of a set (see mm_ld): A0, B0 .. B7, A1 .. A(MB-1), with
// A pieces numbered 0 .. MB-1 and B pieces MB .. MB+7.
struct ReadOrder {
  int v[16];
};
template <int MB>
constexpr ReadOrder read_order() {
  ReadOrder r{};
  r.v[0] = 0;
  for (int i = 1; i <= 8; ++i) r.v[i] = MB + i - 1;
  for (int i = 9; i < MB + 8; ++i) r.v[i] = i - 8;
  return r;
}

// MB: 16-row MFMA blocks per wave along M -- 8 (the 256 x 256 tile) or 4 (a
// 128 x 256 tile: for a product whose 256 x 256 tiles would occupy at most
// half the CUs, twice the workgroups with half the work each).
template <typename T, int EPI, bool AKM, bool BKM, int MB = 8>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_tiled_kernel(GemmArgs args) {
  static_assert(EPI == 0 || (!AKM && !BKM), "the SwiGLU and RoPE epilogues take NT operands");
  static_assert(MB == 8 || (MB == 4 && EPI == 0 && !AKM), "128-row tiles: plain epilogue, A along K");
  constexpr int TBM = 32 * MB;  // tile rows
  constexpr int WR = 16 * MB;   // rows per wave
  const T* __restrict__ A = static_cast<const T*>(args.a);
  const T* __restrict__ B = static_cast<const T*>(args.b);
  const int64_t lda = args.lda, ldb = args.ldb;
  const int64_t M = args.M, N = args.N, K = args.K;
  typedef Mfma<T> Mm;
  typedef typename Mm::vec8 V8;
  __shared__ __attribute__((aligned(16))) T As[3 * TBM * BK];  // ring of three
  __shared__ __attribute__((aligned(16))) T Bs0[BN * BK];
  __shared__ __attribute__((aligned(16))) T Bs1[BN * BK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, q4 = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t n_m = M / TBM, n_n = N / BN, nwg = n_m * n_n;
  int64_t pid = blockIdx.x;
  if ((nwg & 7) == 0) pid = (pid & 7) * (nwg >> 3) + (pid >> 3);
  const int64_t per_group = static_cast<int64_t>(GROUP_M) * n_n;
  const int64_t grp = pid / per_group;
  const int64_t mf = grp * GROUP_M;
  const int64_t gm = n_m - mf < GROUP_M ? n_m - mf : GROUP_M;
  const int64_t in_grp = pid - grp * per_group;
  const int64_t m0 = (mf + in_grp % gm) * TBM, n0 = (in_grp / gm) * BN;
  // first element of the tile and the step between K steps, per layout
  const T* Ab = AKM ? A + m0 : A + m0 * lda;
  const T* Bb = BKM ? B + n0 : B + n0 * ldb;
  const int64_t a_step = AKM ? BK * lda : BK, b_step = BKM ? BK * ldb : BK;
  // EPI 1: the tile's 128 features f0 .. f0 + 127 of both halves.  Tile row
  // block b (16 rows) holds, for wave half wn = b / 8 and jj = b % 8, the gate
  // (jj even) or up (jj odd) rows of features f0 + 64 wn + 16 (jj / 2) ..
  // +15, so a lane's MFMA blocks jj and jj + 1 are g and u of one element.
  const int64_t f0 = n0 / 2;
  // EPI 1: piece p of wave w holds rows 8 (w % 2) .. +7 of features
  // f0 + 16 p .. +15, gate rows for waves 0, 1 and up rows for waves 2, 3
  // (row block 2 p + w / 2); the wave's first source row, kept scalar
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const T* bwave = EPI == 1 ? static_cast<const T*>((wv >> 1) ? args.b2 : args.b) +
                                  (f0 + 8 * (wv & 1)) * ldb
                            : B;

  TileDma<T> adma, bdma;
  TileDmaK<T> admak, bdmak;
  if constexpr (AKM)
    admak.init(lda);
  else
    adma.init(lda);
  if constexpr (BKM)
    bdmak.init(ldb);
  else
    bdma.init(ldb);
  f32x4 acc[MB][8];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{};
  // Operand bases.  NT tiles: lane l reads row l % 16 of each 16-row block,
  // 16-byte chunk l / 16 (substep s: chunk XOR 4 s); nt_sw depends on the row
  // modulo 16 only, so block r of substep s is at ntbase[s] + 1024 r (an
  // immediate offset of the read).  K-major tiles: one base per operand, see
  // kmaj_base.
  int ntA[2] = {0, 0}, ntB[2] = {0, 0};
  int abase = 0, bbase = 0;
  if constexpr (AKM) {
    abase = kmaj_base(wm * WR);
  } else {
    ntA[0] = nt_off(wm * WR + l16, 8 * q4);
    ntA[1] = ntA[0] ^ 32;
  }
  if constexpr (BKM) {
    bbase = kmaj_base(wn * 128);
  } else {
    ntB[0] = nt_off(wn * 128 + l16, 8 * q4);
    ntB[1] = ntB[0] ^ 32;
  }
  V8 xa[2][MB], xb[2][8];
  auto Bs = [&](int st) __attribute__((always_inline)) -> T* { return st ? Bs1 : Bs0; };
  // operand piece r (0..7: A row blocks, 8..15: B row blocks) of substep s
  // into set q
  auto rd_piece = [&](int sa, int sb, int s, int q, int r) __attribute__((always_inline)) {
    if (r < MB) {
      const T* t = &As[sa * (TBM * BK)];
      if constexpr (AKM)
        xa[q][r] = kmaj_operand<T>(t, (abase ^ (16 * r)) + 8192 * s);
      else
        xa[q][r] = *reinterpret_cast<const V8*>(&t[ntA[s] + 1024 * r]);
    } else {
      const T* t = Bs(sb);
      if constexpr (BKM)
        xb[q][r - MB] = kmaj_operand<T>(t, (bbase ^ (16 * (r - MB))) + 8192 * s);
      else
        xb[q][r - MB] = *reinterpret_cast<const V8*>(&t[ntB[s] + 1024 * (r - MB)]);
    }
  };
  auto loadA = [&](int sa, int64_t k, int p) __attribute__((always_inline)) {
    if constexpr (AKM)
      admak.issue(&As[sa * (TBM * BK)], Ab + k * a_step, lda, p);
    else
      adma.issue(&As[sa * (TBM * BK)], Ab + k * a_step, lda, p);
  };
  auto loadB = [&](int sb, int64_t k, int p) __attribute__((always_inline)) {
    if constexpr (EPI != 1) {
      if constexpr (BKM)
        bdmak.issue(Bs(sb), Bb + k * b_step, ldb, p);
      else
        bdma.issue(Bs(sb), Bb + k * b_step, ldb, p);
    } else {
      bdma.issue_wave_rows(Bs(sb), bwave + k * BK,
                           static_cast<uint32_t>(16 * p * ldb * static_cast<int64_t>(sizeof(T))), p);
    }
  };
  // The 8 MB MFMAs of set q in rows of eight.  After row c: A piece c (LK 1:
  // of step k into ring stage lst) or 8 / MB B pieces (LK 2: into B stage
  // lst), and, when RD, (MB + 8) / MB operand pieces of substep s0 of stages
  // (ra, rb) into set q0, in the order the next set's MFMAs use them: its
  // first row needs A piece 0 and all eight B pieces, row c A piece c, so the
  // reads go A0, B0 .. B7, A1 .. A(MB-1) (for MB = 8, B7 is in flight from
  // row 4, three rows before it is needed; read last, it stalled the next
  // set's first MFMA for the LDS latency at every substep).  The fences keep
  // this order.
  constexpr ReadOrder kRO = read_order<MB>();
  constexpr int RPR = (MB + 8) / MB, BPR = 8 / MB;
  auto mm_ld = [&](int q, int lk, int lst, int64_t k, bool rd, int ra, int rb, int s0,
                   int q0) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < MB; ++c) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[c][j] = Mm::mma16(xa[q][c], xb[q][j], acc[c][j]);
      if (rd) {
#pragma unroll
        for (int u = 0; u < RPR; ++u) rd_piece(ra, rb, s0, q0, kRO.v[RPR * c + u]);
      }
      if (lk == 1) loadA(lst, k, c);
      if (lk == 2) {
#pragma unroll
        for (int u = 0; u < BPR; ++u) loadB(lst, k, BPR * c + u);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  const int64_t n_k = K / BK;  // even, >= 4
  // prologue: steps 0 and 1 of A and B
#pragma unroll
  for (int p = 0; p < MB; ++p) loadA(0, 0, p);
#pragma unroll
  for (int p = 0; p < 8; ++p) loadB(0, 0, p);
#pragma unroll
  for (int p = 0; p < MB; ++p) loadA(1, 1, p);
#pragma unroll
  for (int p = 0; p < 8; ++p) loadB(1, 1, p);
  wait_vmcnt<MB + 8>();  // step 0 landed (step 1's MB + 8 loads may be in flight)
  __syncthreads();
#pragma unroll
  for (int r = 0; r < MB + 8; ++r) rd_piece(0, 0, 0, 0, r);

  // K step t: A ring stage sa = t % 3, B stage sb = t % 2; set s = substep s.
  // Part A: set 0 with A(t + 2) (into ring stage (t + 2) % 3, free since the
  // previous barrier) and the reads of substep 1.  Part B: barrier (A(t + 1)
  // and B(t + 1) landed everywhere; this step's reads done), then set 1 with
  // B(t + 2) into B stage sb and the reads of step t + 1's substep 0.  The
  // loop starts at a part B.
  int sa = 0;
  auto partA = [&](auto sb_tag, auto la_tag, int64_t t) __attribute__((always_inline)) {
    constexpr int sb = decltype(sb_tag)::value;
    constexpr bool LA = decltype(la_tag)::value;
    const int sa2 = sa == 0 ? 2 : sa - 1;
    mm_ld(0, LA ? 1 : 0, sa2, t + 2, true, sa, sb, 1, 1);
  };
  // VM8: A(t + 2) was issued in the part A before, and may stay in flight
  auto partB = [&](auto sb_tag, auto sync_tag, auto vm_tag, auto lb_tag, int64_t t) __attribute__((always_inline)) {
    constexpr int sb = decltype(sb_tag)::value;
    constexpr bool SYNC = decltype(sync_tag)::value, VM8 = decltype(vm_tag)::value,
                   LB = decltype(lb_tag)::value;
    const int sa1 = sa == 2 ? 0 : sa + 1;
    if constexpr (SYNC) {
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      if constexpr (VM8)
        wait_vmcnt<MB>();
      else
        wait_vmcnt<0>();
      __syncthreads();
      mm_ld(1, LB ? 2 : 0, sb, t + 2, true, sa1, sb ^ 1, 0, 0);
    } else {
      mm_ld(1, 0, 0, 0, false, 0, 0, 0, 0);
    }
    sa = sa1;
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using BT = std::true_type;
  using BF = std::false_type;
  partA(I0{}, BT{}, 0);
  int64_t kt = 0;
  for (; kt + 4 < n_k; kt += 2) {
    partB(I0{}, BT{}, BT{}, BT{}, kt);
    partA(I1{}, BT{}, kt + 1);
    partB(I1{}, BT{}, BT{}, BT{}, kt + 1);
    partA(I0{}, BT{}, kt + 2);
  }
  partB(I0{}, BT{}, BT{}, BT{}, kt);
  partA(I1{}, BT{}, kt + 1);
  partB(I1{}, BT{}, BT{}, BT{}, kt + 1);
  partA(I0{}, BF{}, kt + 2);
  partB(I0{}, BT{}, BF{}, BF{}, kt + 2);
  partA(I1{}, BF{}, kt + 3);
  partB(I1{}, BF{}, BF{}, BF{}, kt + 3);

  // Epilogue, per wave and 16-row block: the fp32 [16][128] block through the
  // wave's own LDS region (pitch 132 floats), then 16-byte row stores.
  // Accumulator layout: acc[i][j][e] is row 16 i + 4 (l / 16) + e, column
  // 16 j + l % 16 of the wave's block.
  __syncthreads();
  int el = lane;
  asm volatile("" : "+v"(el));  // keep the epilogue's index math after the loop
  // each wave's 16 x 132-float staging area (and for EPI 1 the z tile after
  // it): a 32 KB A stage each for 256-row tiles (Bs0 for wave 3); for 128-row
  // tiles (EPI 0 only) two in the 48 KB A ring, Bs0 and Bs1
  float* ws;
  if constexpr (MB == 8)
    ws = reinterpret_cast<float*>(wave < 3 ? &As[wave * (TBM * BK)] : Bs0);
  else
    ws = wave < 2 ? reinterpret_cast<float*>(As) + wave * (16 * 132)
                  : reinterpret_cast<float*>(wave == 2 ? Bs0 : Bs1);
  const int e16 = el & 15, eq = el >> 4;
  typedef T T8 __attribute__((ext_vector_type(8)));
  // EPI 2: the wave's 128 columns hold whole heads (head dim 2 rhalf = 64 or
  // 128); q / k columns (below rcols) are rotated, v columns stored as is.
  // Sequence position of the wave's first row; a row 16 i + r further is at
  // (rs0 + 16 i + r) mod rS (32-bit: the host keeps rS in [128, 2^30)).
  const bool rot = EPI == 2 && n0 + wn * 128 < args.rcols;
  const int rs32 = static_cast<int>(args.rS);
  const int rs0 = EPI == 2 ? static_cast<int>((m0 + wm * WR) % args.rS) : 0;
  auto rope_pos = [&](int off) -> int {
    int sq = rs0 + off;
    sq = sq >= rs32 ? sq - rs32 : sq;  // the host takes this path for rS >= 128 only
    int64_t pos = args.rpos != nullptr ? args.rpos[sq] : sq;
    pos = pos < 0 ? 0 : pos > args.rnpos - 1 ? args.rnpos - 1 : pos;
    return static_cast<int>(pos) * args.rhalf;  // table offset (host: positions below 2^24)
  };
  // half-split pairing: 8-column chunks per half head, 2^hcl (8 for head dim
  // 128, 4 for 64)
  const int hcl = args.rhalf == 64 ? 3 : 2, hcm = (1 << hcl) - 1;
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    // EPI 2, half-split pairing: this block's cos / sin, loaded before the
    // staging stores below so that their latency overlaps them
    float4 rc0[2], rc1[2], rsn0[2], rsn1[2];
    if (EPI == 2 && rot && args.rpair == ZK_ROPE_HALF) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int it = q * 64 + el;
        const int toff = rope_pos(16 * i + (it >> 3)) + 8 * ((it & 7) & hcm);
        const float* cp = args.rcos + toff;
        const float* sp = args.rsin + toff;
        rc0[q] = *reinterpret_cast<const float4*>(cp);
        rc1[q] = *reinterpret_cast<const float4*>(cp + 4);
        rsn0[q] = *reinterpret_cast<const float4*>(sp);
        rsn1[q] = *reinterpret_cast<const float4*>(sp + 4);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) ws[(4 * eq + e) * 132 + 16 * j + e16] = acc[i][j][e];
    const int64_t row0 = m0 + wm * WR + 16 * i;
    if (EPI == 2 && rot && args.rpair == ZK_ROPE_HALF) {
      // 16 rows x 8 chunk pairs: chunk a (first half of its head) with the
      // chunk rhalf / 8 further; the product rounded to T first, as stored
      T* C = static_cast<T*>(args.c);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int it = q * 64 + el;
        const int rr = it >> 3, pc = it & 7;
        // chunks per half head hc = 2^hcl (4 or 8)
        const int ca = ((pc >> hcl) << (hcl + 1)) + (pc & hcm), cb = ca + (1 << hcl);
        const int64_t grow = row0 + rr;
        const float cs[8] = {rc0[q].x, rc0[q].y, rc0[q].z, rc0[q].w,
                             rc1[q].x, rc1[q].y, rc1[q].z, rc1[q].w};
        const float sn[8] = {rsn0[q].x, rsn0[q].y, rsn0[q].z, rsn0[q].w,
                             rsn1[q].x, rsn1[q].y, rsn1[q].z, rsn1[q].w};
        T8 o1, o2;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x1 = round_to<T>(ws[rr * 132 + 8 * ca + e]);
          const float x2 = round_to<T>(ws[rr * 132 + 8 * cb + e]);
          float y1, y2;
          rotate_pair<T, ZK_ROPE_HALF, false>(x1, x2, cs[e], sn[e], y1, y2);
          o1[e] = static_cast<T>(y1);
          o2[e] = static_cast<T>(y2);
        }
        const int64_t gcol = n0 + wn * 128;
        *reinterpret_cast<T8*>(C + grow * args.ldc + gcol + 8 * ca) = o1;
        *reinterpret_cast<T8*>(C + grow * args.ldc + gcol + 8 * cb) = o2;
      }
    } else if (EPI == 2 && rot) {
      // interleaved pairs (2 i, 2 i + 1) inside each chunk: 16 rows x 16 chunks
      T* C = static_cast<T*>(args.c);
      const int cpm = (args.rhalf >> 2) - 1;  // chunks per head (8 or 16), less one
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = q * 64 + el;
        const int rr = c >> 4, ch = c & 15;
        const int64_t grow = row0 + rr;
        const int toff = rope_pos(16 * i + rr) + 4 * (ch & cpm);  // the chunk's first pair
        const float4 cv = *reinterpret_cast<const float4*>(args.rcos + toff);
        const float4 sv = *reinterpret_cast<const float4*>(args.rsin + toff);
        const float cs[4] = {cv.x, cv.y, cv.z, cv.w}, sn[4] = {sv.x, sv.y, sv.z, sv.w};
        T8 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x1 = round_to<T>(ws[rr * 132 + 8 * ch + 2 * j]);
          const float x2 = round_to<T>(ws[rr * 132 + 8 * ch + 2 * j + 1]);
          float y1, y2;
          rotate_pair<T, ZK_ROPE_INTERLEAVED, false>(x1, x2, cs[j], sn[j], y1, y2);
          o[2 * j] = static_cast<T>(y1);
          o[2 * j + 1] = static_cast<T>(y2);
        }
        *reinterpret_cast<T8*>(C + grow * args.ldc + n0 + wn * 128 + 8 * ch) = o;
      }
    } else if constexpr (EPI != 1) {
      // c = acc (+ r), one rounding; 16 rows x 16 chunks of 8 columns
      T* C = static_cast<T*>(args.c);
      const T* R = static_cast<const T*>(args.r);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = q * 64 + el;
        const int rr = c >> 4, ch = c & 15;
        const float4 lo = *reinterpret_cast<const float4*>(&ws[rr * 132 + 8 * ch]);
        const float4 hi = *reinterpret_cast<const float4*>(&ws[rr * 132 + 8 * ch + 4]);
        float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        const int64_t grow = row0 + rr;
        const int64_t gcol = n0 + wn * 128 + 8 * ch;
        if (R != nullptr) {
          const T8 rv = *reinterpret_cast<const T8*>(R + grow * args.ldr + gcol);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] += to_f32(rv[e]);
        }
        T8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = static_cast<T>(v[e]);
        *reinterpret_cast<T8*>(C + grow * args.ldc + gcol) = o;
      }
    } else {
      // g, u rounded as the GEMM would store them; z = round(round(silu(g)) u)
      // (the SwiGLU kernel's rounding points); z also into a feature-major
      // tile of the wave's 128 tokens (pitch 136), stored transposed after
      // the last block in whole 256-byte rows.  Columns 32 jp + 8 h of the
      // staged block are gate features 16 jp + 8 h, 16 further the up ones.
      T* G = static_cast<T*>(args.c);
      T* U = static_cast<T*>(args.c2);
      T* Z = static_cast<T*>(args.z);
      T* zs = reinterpret_cast<T*>(ws + 16 * 132);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int it = q * 64 + el;
        const int rr = it >> 3, jp = (it >> 1) & 3, h = it & 1;
        const float* gp = &ws[rr * 132 + 32 * jp + 8 * h];
        const float4 g0 = *reinterpret_cast<const float4*>(gp);
        const float4 g1 = *reinterpret_cast<const float4*>(gp + 4);
        const float4 u0 = *reinterpret_cast<const float4*>(gp + 16);
        const float4 u1 = *reinterpret_cast<const float4*>(gp + 20);
        const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        const float uv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
        T8 go, uo, zo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          go[e] = static_cast<T>(gv[e]);
          uo[e] = static_cast<T>(uv[e]);
          zo[e] = static_cast<T>(round_to<T>(silu_fast(to_f32(go[e]))) * to_f32(uo[e]));
          zs[(16 * jp + 8 * h + e) * 136 + 16 * i + rr] = zo[e];
        }
        const int64_t grow = row0 + rr;
        const int64_t f = f0 + wn * 64 + 16 * jp + 8 * h;
        *reinterpret_cast<T8*>(G + grow * args.ldc + f) = go;
        *reinterpret_cast<T8*>(U + grow * args.ldc + f) = uo;
        *reinterpret_cast<T8*>(Z + grow * args.ldz + f) = zo;
      }
    }
  }
  if constexpr (EPI == 1) {
    if (args.zt != nullptr) {
      // 64 feature rows x 16 chunks of 8 tokens (the wave's 128 tokens)
      T* ZT = static_cast<T*>(args.zt);
      const T* zs = reinterpret_cast<const T*>(ws + 16 * 132);
      const int64_t fw0 = f0 + wn * 64, t0 = m0 + wm * 128;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int ch = q * 64 + el;
        const int fr = ch >> 4, tc = ch & 15;
        const T8 v = *reinterpret_cast<const T8*>(&zs[fr * 136 + 8 * tc]);
        *reinterpret_cast<T8*>(ZT + (fw0 + fr) * args.ldzt + t0 + 8 * tc) = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Any shape and layout, bf16 / fp16 / fp32: 4 waves, a 128 x 128 tile (each
// wave 64 x 64 as 4 x 4 MFMA blocks), K steps of 32.  Each step's operand
// tiles are read from global memory into registers with every index checked
// (out-of-range elements are zero), written to LDS as [128 rows][32 k] (k
// contiguous, padded rows), and consumed by v_mfma_f32_16x16x32 (2-byte
// types) or v_mfma_f32_16x16x4f32 (fp32, full fp32 products).  Stores are
// masked per element.  This is the path for token counts off the 256 grid
// and for fp32 layers; it needs no alignment beyond the element's.
constexpr int GBM = 128, GBK = 32;

template <typename T>
struct GenCfg {
  static constexpr int P = sizeof(T) == 2 ? GBK + 8 : GBK + 4;  // LDS row pitch (elements)
};

// One [128][32] operand tile (rows r0 .., k0 ..) into LDS at `t` (pitch P).
// KM: the operand is stored [K][rows]; else [rows][K].
template <typename T, bool KM>
__device__ __forceinline__ void gen_stage(T* t, const T* __restrict__ src, int64_t ld, int64_t r0,
                                          int64_t R, int64_t k0, int64_t K) {
  constexpr int P = GenCfg<T>::P;
  const int tid = threadIdx.x;
  T v[16];
  if constexpr (!KM) {
    // thread: row tid / 2, 16 consecutive k from 16 (tid % 2)
    const int r = tid >> 1, kk = (tid & 1) * 16;
    const int64_t gr = r0 + r;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int64_t gk = k0 + kk + e;
      v[e] = (gr < R && gk < K) ? src[gr * ld + gk] : static_cast<T>(0.0f);
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) t[r * P + kk + e] = v[e];
  } else {
    // thread: k = tid / 8, 16 consecutive rows from 16 (tid % 8)
    const int k = tid >> 3, rr = (tid & 7) * 16;
    const int64_t gk = k0 + k;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int64_t gr = r0 + rr + e;
      v[e] = (gr < R && gk < K) ? src[gk * ld + gr] : static_cast<T>(0.0f);
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) t[(rr + e) * P + k] = v[e];
  }
}

template <typename T, bool AKM, bool BKM>
__global__ __launch_bounds__(256) void gemm_gen_kernel(GemmArgs args) {
  constexpr int P = GenCfg<T>::P;
  __shared__ __attribute__((aligned(16))) T As[GBM * P];
  __shared__ __attribute__((aligned(16))) T Bs[GBM * P];
  const T* __restrict__ A = static_cast<const T*>(args.a);
  const T* __restrict__ B = static_cast<const T*>(args.b);
  const int64_t M = args.M, N = args.N, K = args.K;
  const int64_t n_n = (N + GBM - 1) / GBM;
  const int64_t m0 = (blockIdx.x / n_n) * GBM, n0 = (blockIdx.x % n_n) * GBM;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1, l16 = lane & 15, q4 = lane >> 4;
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{};
  for (int64_t k0 = 0; k0 < K; k0 += GBK) {
    gen_stage<T, AKM>(As, A, args.lda, m0, M, k0, K);
    gen_stage<T, BKM>(Bs, B, args.ldb, n0, N, k0, K);
    __syncthreads();
    if constexpr (sizeof(T) == 2) {
      typedef typename Mfma<T>::vec8 V8;
      V8 xa[4], xb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xa[i] = *reinterpret_cast<const V8*>(&As[(wm * 64 + 16 * i + l16) * P + 8 * q4]);
        xb[i] = *reinterpret_cast<const V8*>(&Bs[(wn * 64 + 16 * i + l16) * P + 8 * q4]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = Mfma<T>::mma16(xa[i], xb[j], acc[i][j]);
    } else {
      // lane l: row l % 16, k = 4 kk + l / 16
#pragma unroll
      for (int kk = 0; kk < GBK / 4; ++kk) {
        float xa[4], xb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          xa[i] = As[(wm * 64 + 16 * i + l16) * P + 4 * kk + q4];
          xb[i] = Bs[(wn * 64 + 16 * i + l16) * P + 4 * kk + q4];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[i], xb[j], acc[i][j], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  // acc[i][j][e]: row 16 i + 4 (l / 16) + e, column 16 j + l % 16 of the
  // wave's 64 x 64 block
  T* C = static_cast<T*>(args.c);
  const T* R = static_cast<const T*>(args.r);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t row = m0 + wm * 64 + 16 * i + 4 * q4 + e;
        const int64_t col = n0 + wn * 64 + 16 * j + l16;
        if (row < M && col < N) {
          float v = acc[i][j][e];
          if (R != nullptr) v += to_f32(R[row * args.ldr + col]);
          C[row * args.ldc + col] = static_cast<T>(v);
        }
      }
}

// The tiled kernel with A and / or B K-major (gemm_kmajor.hip), bf16 or fp16,
// on a launch tiled_takes accepted.
void launch_tiled_kmajor(bool bf16, bool a_kmajor, bool b_kmajor, const GemmArgs& ga,
                         hipStream_t s);

}  // namespace gemm

}  // namespace zk
