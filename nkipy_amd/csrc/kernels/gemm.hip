// MFMA GEMM with fused epilogues for gfx950 (CDNA4).
//
//   plain:   C = A * B (* col_scale) (+ bias) (+ residual)
//   swiglu:  H = silu(A * B0) * (A * B1)   (gate and up tiles in one kernel)
//
// A is M x K row-major bf16 (K contiguous).  B is either
//   NN: K x N row-major (N contiguous)  -- x @ W with W (in, out), as in
//       examples/models/qwen3/kernels/feedforward.py:9-18, or
//   NT: N x K row-major (K contiguous)  -- x @ W.T with W (out, in), the torch
//       Linear layout of tests/kernels/mlp_dynamo.py:9-25.
// B elements are bf16 or fp8 E4M3FN; fp8 is widened to bf16 exactly while
// staging into LDS and its per-output-column scale is applied in the epilogue
// (W8A16: bf16 MFMA on exact dequantised weights, fp32 accumulation).
//
// Tiling: 256 threads = 4 waves (2 x 2).  Block tile 256 (M) x 256 (N cols of
// B) x 64 (K); each wave owns 128 x 128 = 4 x 4 tiles of
// v_mfma_f32_32x32x16_bf16 (256 fp32 accumulators per lane).  In swiglu mode
// the 256 B columns are 128 gate + 128 up columns of the same output columns,
// and each wave holds matching gate / up tiles so the epilogue combines them
// in registers.  LDS holds two stages of A[256][64] and B^T[256][64] (bf16,
// K contiguous, 16-byte chunks XOR-swizzled by row) = 128 KiB; the next K
// tile is fetched into registers while the current one feeds the MFMAs.
// NN weights are transposed in registers (8 x 8 bf16 blocks) on the way into
// LDS, so both layouts are read by the MFMA loop identically.
// Work distribution is XCD aware: consecutive workgroup ids are dealt to the
// 8 XCDs round robin, so ids are remapped so that each XCD receives a
// contiguous run of tiles, walked in groups of GROUP_M tile rows.

#include "common.h"

using namespace nk;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

#define BM 256
#define BN 256
#define BK 64
#define NTHREADS 256
#define GROUP_M 8

enum {
  GEMM_BIAS = 1,      // + bias[col] (bf16)
  GEMM_SCALE = 2,     // * scale[col] (fp32), per output column (fp8 weights)
  GEMM_RESID = 4,     // + residual[row][col] (same dtype as C)
  GEMM_VEC = 8,       // C / residual rows allow aligned 4-element vector access
};

struct GemmArgs {
  const void *A;       // M x K
  const void *B0;      // NN: K x N ; NT: N x K
  const void *B1;      // swiglu: up weight (same layout as B0)
  void *C;             // M x N (swiglu: M x N_out)
  const void *bias;    // N, bf16
  const float *scale0; // N, fp32 (scales of B0 columns)
  const float *scale1; // N, fp32 (scales of B1 columns, swiglu)
  const void *resid;   // M x N, C dtype
  int64_t M, N, K;     // N = output columns
  int64_t lda, ldb, ldc;
  int32_t tiles_m, tiles_n;
  int32_t flags, pad;
};

// ---------------------------------------------------------------------------
// element helpers
// ---------------------------------------------------------------------------
// fp8 -> bf16 staging uses nk::e4m3x8_to_bf16x8 (common.h)

template <typename TC> struct OutT;
template <> struct OutT<bf16> {
  static __device__ __forceinline__ void store(void *C, int64_t i, float v) {
    reinterpret_cast<uint16_t *>(C)[i] = f32_to_bf16(v);
  }
  static __device__ __forceinline__ float load(const void *C, int64_t i) {
    return bf16_to_f32(reinterpret_cast<const uint16_t *>(C)[i]);
  }
  static __device__ __forceinline__ void store4(void *C, int64_t i, const float (&v)[4]) {
    *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(C) + i) =
        make_uint2((uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16),
                   (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16));
  }
  static __device__ __forceinline__ void load4(const void *C, int64_t i, float (&v)[4]) {
    const uint2 w = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(C) + i);
    v[0] = __uint_as_float(w.x << 16);
    v[1] = __uint_as_float(w.x & 0xffff0000u);
    v[2] = __uint_as_float(w.y << 16);
    v[3] = __uint_as_float(w.y & 0xffff0000u);
  }
};
template <> struct OutT<float> {
  static __device__ __forceinline__ void store(void *C, int64_t i, float v) {
    reinterpret_cast<float *>(C)[i] = v;
  }
  static __device__ __forceinline__ float load(const void *C, int64_t i) {
    return reinterpret_cast<const float *>(C)[i];
  }
  static __device__ __forceinline__ void store4(void *C, int64_t i, const float (&v)[4]) {
    *reinterpret_cast<float4 *>(reinterpret_cast<float *>(C) + i) = make_float4(v[0], v[1], v[2], v[3]);
  }
  static __device__ __forceinline__ void load4(const void *C, int64_t i, float (&v)[4]) {
    const float4 w = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(C) + i);
    v[0] = w.x;
    v[1] = w.y;
    v[2] = w.z;
    v[3] = w.w;
  }
};

// half-word i (0..7) of an 8 x bf16 vector
__device__ __forceinline__ uint32_t h16(const uint4 &v, int i) {
  uint32_t w = (i < 2) ? v.x : (i < 4) ? v.y : (i < 6) ? v.z : v.w;
  return (i & 1) ? (w >> 16) : (w & 0xffffu);
}

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// ---------------------------------------------------------------------------
// global -> LDS movement
// ---------------------------------------------------------------------------
// Operands are read through buffer resources: 32-bit offsets from one base
// (no per-load 64-bit addresses), and an offset past the end (OOB) reads
// zeros, which pads the M / N / K edges without branches.
#define OOB 0x80000000u
#define BUF_WORD3 0x00020000  // gfx9 buffer resource word 3 (raw, untyped)

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, BUF_WORD3);
}

// One wave moves 1 KiB: lane l's 16 bytes land at lds_block + 16 * l.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t *lds_block, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds_block, 16, off, 0, 0, 0);
}

// Each thread's DMA sources are fixed up to the K offset: per 16-byte move j
// the byte offset at k0 = 0 (OOB if its row / column is outside the matrix)
// and the K index of its chunk.  Per K tile: off = base + k0 * kstep, or OOB
// past K.  Wave index `wave` is wave-uniform (scalar), so the LDS block
// addresses (M0) are scalar too.
template <int NJ>
struct DmaPlan {
  uint32_t base[NJ];
  int kofs;  // chunk K index common to all j (row-major operands), else per j below
};

__device__ __forceinline__ uint32_t dma_off(uint32_t base, int64_t k0, int kidx, int64_t K, int64_t kstep) {
  return (base != OOB && k0 + kidx < K) ? base + (uint32_t)(k0 * kstep) : OOB;
}

// A tile (and a bf16 B^T tile): 256 rows x 64 bf16 = 128-byte rows, 16-byte
// chunks stored at chunk ^ swz(row).  Wave w moves blocks b = 4 j + w of
// 8 rows; lane l fills stored slot (row, l % 8), so it fetches logical chunk
// (l % 8) ^ swz(row) -- the same chunk for every j, since swz(row) only
// depends on (4 w + l / 16) mod 8.
__device__ __forceinline__ DmaPlan<8> plan_rows_bf16(bool split, int64_t r_first, int64_t nrows, int64_t ld,
                                                     int wave, int lane) {
  DmaPlan<8> p;
  const int lc = (lane & 7) ^ swz(wave * 8 + (lane >> 3), 0);  // row of move j = 0
  p.kofs = lc * 8;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int b = j * 4 + wave;
    const int row = b * 8 + (lane >> 3);
    const int64_t rr = r_first + ((split && b >= 16) ? row - 128 : row);
    p.base[j] = rr < nrows ? (uint32_t)((rr * ld + p.kofs) * 2) : OOB;
  }
  return p;
}

__device__ __forceinline__ void dma_rows_bf16(const DmaPlan<8> &p, __amdgpu_buffer_rsrc_t r0,
                                              __amdgpu_buffer_rsrc_t r1, bool split, uint8_t *S, int64_t k0,
                                              int64_t K, int wave) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int b = j * 4 + wave;
    dma16((split && b >= 16) ? r1 : r0, S + b * 1024, dma_off(p.base[j], k0, p.kofs, K, 2));
  }
}

// fp8 B^T tile (NT weights): 256 rows x 64 codes = 64-byte rows, 16-byte
// chunks stored at chunk ^ ((row >> 2) & 3).  Blocks of 16 rows.
__device__ __forceinline__ int swz8(int row) { return (row >> 2) & 3; }

__device__ __forceinline__ DmaPlan<4> plan_rows_fp8(bool split, int64_t r_first, int64_t nrows, int64_t ld,
                                                    int wave, int lane) {
  DmaPlan<4> p;
  const int lc = (lane & 3) ^ swz8(wave * 16 + (lane >> 2));  // row of move j = 0
  p.kofs = lc * 16;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int b = j * 4 + wave;
    const int row = b * 16 + (lane >> 2);
    const int64_t rr = r_first + ((split && b >= 8) ? row - 128 : row);
    p.base[j] = rr < nrows ? (uint32_t)(rr * ld + p.kofs) : OOB;
  }
  return p;
}

__device__ __forceinline__ void dma_rows_fp8(const DmaPlan<4> &p, __amdgpu_buffer_rsrc_t r0,
                                             __amdgpu_buffer_rsrc_t r1, bool split, uint8_t *S, int64_t k0,
                                             int64_t K, int wave) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int b = j * 4 + wave;
    dma16((split && b >= 8) ? r1 : r0, S + b * 1024, dma_off(p.base[j], k0, p.kofs, K, 1));
  }
}

// bf16 NN B tile (K x N weights, N contiguous): stored as two column halves
// [64 k][128 n] with 256-byte rows (half 0 = tile columns 0..127, half 1 =
// 128..255; in SwiGLU mode gate and up), 16-byte chunks at chunk ^ nnswz(k).
// MFMA fragments are read with ds_read_b64_tr_b16 (below).  Blocks of 4 rows;
// move j covers k row ((4 j + w) mod 16) * 4 + l / 16.
__device__ __forceinline__ int nnswz(int k) { return (k & 3) << 2; }

__device__ __forceinline__ int nn_krow(int j, int wave, int lane) { return ((j * 4 + wave) & 15) * 4 + (lane >> 4); }

__device__ __forceinline__ DmaPlan<8> plan_nn_bf16(bool split, int64_t n0, int64_t N, int64_t ld, int wave,
                                                   int lane) {
  DmaPlan<8> p;
  p.kofs = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int b = j * 4 + wave;
    const int half = b >> 4;
    const int k = nn_krow(j, wave, lane);
    const int lc = (lane & 15) ^ nnswz(k);
    const int64_t col = n0 + (split ? 0 : half * 128) + lc * 8;
    p.base[j] = col < N ? (uint32_t)((k * ld + col) * 2) : OOB;
  }
  return p;
}

__device__ __forceinline__ void dma_nn_bf16(const DmaPlan<8> &p, __amdgpu_buffer_rsrc_t r0,
                                            __amdgpu_buffer_rsrc_t r1, bool split, uint8_t *S, int64_t k0,
                                            int64_t K, int64_t ld, int wave, int lane) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int b = j * 4 + wave;
    dma16((split && (b >> 4)) ? r1 : r0, S + b * 1024,
          dma_off(p.base[j], k0, nn_krow(j, wave, lane), K, ld * 2));
  }
}

// NN weights (K x N, N contiguous) go through registers: thread -> (8 k rows,
// 8 columns); the 8 x 8 block is transposed in registers into B^T rows.
struct StageNN {
  uint4 r[8];
};

template <bool FP8, bool SWIGLU>
__device__ __forceinline__ void load_nn(StageNN &s, const GemmArgs &a, __amdgpu_buffer_rsrc_t r0,
                                        __amdgpu_buffer_rsrc_t r1, int64_t n0, int64_t k0) {
  const int kb = threadIdx.x >> 5, nc = threadIdx.x & 31;
  const bool second = SWIGLU && nc >= 16;
  const int64_t col = n0 + (SWIGLU ? (nc & 15) * 8 : nc * 8);
  const __amdgpu_buffer_rsrc_t r = second ? r1 : r0;
  uint4 in[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t k = k0 + kb * 8 + j;
    const bool ok = k < a.K && col < a.N;
    if (FP8) {
      const uint32_t off = ok ? (uint32_t)(k * a.ldb + col) : OOB;
      u32x2 q = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
      in[j] = e4m3x8_to_bf16x8(make_uint2(q[0], q[1]));
    } else {
      const uint32_t off = ok ? (uint32_t)((k * a.ldb + col) * 2) : OOB;
      u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
      in[j] = make_uint4(q[0], q[1], q[2], q[3]);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) w[p] = h16(in[2 * p], i) | (h16(in[2 * p + 1], i) << 16);
    s.r[i] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

__device__ __forceinline__ void store_nn(const StageNN &s, uint8_t *Bs) {
  const int kb = threadIdx.x >> 5, nc = threadIdx.x & 31;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int nt = nc * 8 + i;
    *reinterpret_cast<uint4 *>(Bs + nt * 128 + swz(nt, kb) * 16) = s.r[i];
  }
}

__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)
// vmcnt(N): all but the N most recent vector memory loads have completed
// (loads retire in issue order)
template <int N>
__device__ __forceinline__ void wait_vmem_but() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
// Workgroup barrier without __syncthreads()'s release fence, which would
// wait for every outstanding load (vmcnt(0)), including the DMA of the tile
// after next.  Ordering is explicit instead: each wave waits (vmcnt) for the
// DMAs the next tile needs before the barrier, and every LDS read of a stage
// has been consumed by an MFMA before the barrier that precedes the stage's
// refill.  The empty asm statements keep the compiler from moving memory
// accesses across the barrier.
__device__ __forceinline__ void barrier_no_fence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------
// MFMA over one staged K tile (64 = 4 steps of 16), operand fragments of
// step kk + 1 read from LDS while step kk's MFMAs run
// ---------------------------------------------------------------------------
// B staging modes: raw fp8 NT rows, bf16 B^T rows, bf16 NN column halves
enum BMode { B_T16 = 0, B_T8 = 1, B_NN16 = 2 };

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

template <int BM_>
__device__ __forceinline__ void read_frags(bf16x8_t (&af)[4], bf16x8_t (&bf)[4], const uint8_t *As,
                                           const uint8_t *Bs, int kk, int wm, const int (&brow)[4],
                                           int lane) {
  const int l32 = lane & 31, lhi = lane >> 5;
  const int chunk = kk * 2 + lhi;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = wm * 128 + i * 32 + l32;
    af[i] = *reinterpret_cast<const bf16x8_t *>(As + row * 128 + swz(row, chunk) * 16);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (BM_ == B_T8) {
      const int row = brow[j] + l32;
      const uint2 q = *reinterpret_cast<const uint2 *>(Bs + row * 64 + (kk ^ swz8(row)) * 16 + lhi * 8);
      const uint4 w = e4m3x8_to_bf16x8(q);
      bf[j] = *reinterpret_cast<const bf16x8_t *>(&w);
    } else if (BM_ == B_T16) {
      const int row = brow[j] + l32;
      bf[j] = *reinterpret_cast<const bf16x8_t *>(Bs + row * 128 + swz(row, chunk) * 16);
    } else {
      // brow[j] = tile column; half = column / 128.  Lane (group g, index i):
      // source of row k = kk*16 + 8*(g/2) + 4*s + i/4, columns c + 16*(g%2) + 4*(i%4).
      const int half = brow[j] >> 7, c = brow[j] & 127;
      const int g = lane >> 4, i = lane & 15;
      const int nl = c + (g & 1) * 16 + 4 * (i & 3);
      s16x4 v[2];
#pragma unroll
      for (int sidx = 0; sidx < 2; ++sidx) {
        const int k = kk * 16 + (g >> 1) * 8 + 4 * sidx + (i >> 2);
        const uint8_t *p = Bs + half * 16384 + k * 256 + (((nl >> 3) ^ nnswz(k)) << 4) + (nl & 7) * 2;
        v[sidx] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)p);
      }
      bf[j] = __builtin_shufflevector(__builtin_bit_cast(__attribute__((ext_vector_type(4))) __bf16, v[0]),
                                      __builtin_bit_cast(__attribute__((ext_vector_type(4))) __bf16, v[1]),
                                      0, 1, 2, 3, 4, 5, 6, 7);
    }
  }
}

template <int BM_>
__device__ __forceinline__ void mma_tile(f32x16 (&acc)[4][4], const uint8_t *As, const uint8_t *Bs, int wm,
                                         const int (&brow)[4], int lane) {
  bf16x8_t af[2][4], bf[2][4];
  read_frags<BM_>(af[0], bf[0], As, Bs, 0, wm, brow, lane);
#pragma unroll
  for (int kk = 0; kk < BK / 16; ++kk) {
    if (kk + 1 < BK / 16) read_frags<BM_>(af[(kk + 1) & 1], bf[(kk + 1) & 1], As, Bs, kk + 1, wm, brow, lane);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[kk & 1][j], af[kk & 1][i], acc[i][j], 0, 0, 0);
  }
}

// Instruction order of one K tile (one scheduling region: the DMA issue of
// the next tile plus the MFMAs of this one): half of the next tile's DMAs
// first and the other half after the first step's 8 MFMAs, so that each has
// most of the tile's MFMA time to land before the closing vmcnt(0) wait
// (measured best among up-front, spread and split issue); fragments of step
// 0 first, and per step the fragments of step + 1 ahead of the step's 16
// MFMAs, so each read has a whole step (~512 cycles) to land.
template <int NDS, int NVMEM>
__device__ __forceinline__ void schedule_ktile() {
  __builtin_amdgcn_sched_group_barrier(0x020, NVMEM / 2, 0);  // VMEM reads (DMA)
  __builtin_amdgcn_sched_group_barrier(0x100, NDS, 0);        // DS reads, step 0
#pragma unroll
  for (int kk = 0; kk < BK / 16; ++kk) {
    if (kk + 1 < BK / 16) __builtin_amdgcn_sched_group_barrier(0x100, NDS, 0);  // DS reads, step kk + 1
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);                           // 8 MFMA
    if (kk == 0) __builtin_amdgcn_sched_group_barrier(0x020, NVMEM - NVMEM / 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);                           // 8 MFMA
  }
}

// ---------------------------------------------------------------------------
// main kernel
// ---------------------------------------------------------------------------
template <bool NT, bool FP8, bool SWIGLU, typename TC>
__device__ __forceinline__ void gemm_body(const GemmArgs &a) {
  // fp8 NT codes staged raw (decoded per fragment); bf16 NN through LDS DMA
  // and transpose reads; fp8 NN through registers into bf16 B^T rows
  constexpr int BMODE = (NT && FP8) ? B_T8 : (!NT && !FP8) ? B_NN16 : B_T16;
  constexpr bool REG_B = !NT && FP8;
  constexpr int BROW = BMODE == B_T8 ? 64 : 128;  // bytes per B row in LDS

  // XCD-aware tile order
  const int ntiles = a.tiles_m * a.tiles_n;
  int pid = blockIdx.x;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  const int in_group = GROUP_M * a.tiles_n;
  const int group = pid / in_group;
  const int first_m = group * GROUP_M;
  const int gsize = min(a.tiles_m - first_m, GROUP_M);
  const int tm = first_m + (pid % in_group) % gsize;
  const int tn = (pid % in_group) / gsize;
  const int64_t m0 = (int64_t)tm * BM;
  const int64_t n0 = (int64_t)tn * (SWIGLU ? BN / 2 : BN);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // B^T rows read by this wave for tile column block j
  int brow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    brow[j] = SWIGLU ? ((j < 2) ? (wn * 64 + j * 32) : (128 + wn * 64 + (j - 2) * 32))
                     : (wn * 128 + j * 32);

  const int bsz = FP8 ? 1 : 2;
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(a.A, a.M * a.lda * 2);
  const int64_t brows = NT ? a.N : a.K;  // rows of the stored B matrix
  const __amdgpu_buffer_rsrc_t rb0 = make_rsrc(a.B0, brows * a.ldb * bsz);
  const __amdgpu_buffer_rsrc_t rb1 = make_rsrc(SWIGLU ? a.B1 : a.B0, brows * a.ldb * bsz);

  StageNN sn;
  const DmaPlan<8> pa = plan_rows_bf16(false, m0, a.M, a.lda, wave, lane);
  DmaPlan<8> pb16;
  DmaPlan<4> pb8;
  if (NT && FP8) pb8 = plan_rows_fp8(SWIGLU, n0, a.N, a.ldb, wave, lane);
  if (NT && !FP8) pb16 = plan_rows_bf16(SWIGLU, n0, a.N, a.ldb, wave, lane);
  if (!NT && !FP8) pb16 = plan_nn_bf16(SWIGLU, n0, a.N, a.ldb, wave, lane);
  auto issue_a = [&](uint8_t *As, int64_t k0) { dma_rows_bf16(pa, ra, ra, false, As, k0, a.K, wave); };
  auto issue_b = [&](uint8_t *Bs, int64_t k0) {
    if (NT) {
      if (FP8)
        dma_rows_fp8(pb8, rb0, rb1, SWIGLU, Bs, k0, a.K, wave);
      else
        dma_rows_bf16(pb16, rb0, rb1, SWIGLU, Bs, k0, a.K, wave);
    } else if (REG_B) {
      load_nn<FP8, SWIGLU>(sn, a, rb0, rb1, n0, k0);
    } else {
      dma_nn_bf16(pb16, rb0, rb1, SWIGLU, Bs, k0, a.K, a.ldb, wave, lane);
    }
  };
  auto issue = [&](uint8_t *As, uint8_t *Bs, int64_t k0) {
    issue_a(As, k0);
    issue_b(Bs, k0);
  };

  const int ktiles = (int)((a.K + BK - 1) / BK);
  // fragment reads per step and DMA moves per K tile of this variant
  constexpr int NDS = BMODE == B_NN16 ? 12 : 8;
  constexpr int NVM = REG_B ? 16 : (BMODE == B_T8 ? 12 : 16);

  // DMA moves of the B tile per K tile
  constexpr int NVB = BMODE == B_T8 ? 4 : 8;

  if constexpr (BMODE == B_T8) {
    // fp8 B^T: 48 KiB stages, a three-stage ring (144 KiB).  The DMA of tile
    // t + 2 is issued while tile t feeds the MFMAs, and the closing wait only
    // needs tile t + 1 (issued a whole tile earlier), so the DMA latency tail
    // stays off the critical path.  A step past the last tile reads zeros (K
    // offset out of range) into a stage that is never consumed.
    __shared__ __attribute__((aligned(1024))) uint8_t A0[BM * 128];
    __shared__ __attribute__((aligned(1024))) uint8_t A1[BM * 128];
    __shared__ __attribute__((aligned(1024))) uint8_t A2[BM * 128];
    __shared__ __attribute__((aligned(1024))) uint8_t B0[BN * BROW];
    __shared__ __attribute__((aligned(1024))) uint8_t B1[BN * BROW];
    __shared__ __attribute__((aligned(1024))) uint8_t B2[BN * BROW];
    issue(A0, B0, 0);
    issue(A1, B1, BK);
    wait_vmem_but<NVM>();
    barrier_no_fence();
    auto step = [&](uint8_t *Ac, uint8_t *Bc, uint8_t *An, uint8_t *Bn, int tt) __attribute__((always_inline)) {
      issue(An, Bn, (int64_t)(tt + 2) * BK);
      mma_tile<BMODE>(acc, Ac, Bc, wm, brow, lane);
      schedule_ktile<NDS, NVM>();
      wait_vmem_but<NVM>();
      barrier_no_fence();
    };
    int t = 0;
    for (; t + 3 <= ktiles; t += 3) {
      step(A0, B0, A2, B2, t);
      step(A1, B1, A0, B0, t + 1);
      step(A2, B2, A1, B1, t + 2);
    }
    if (t < ktiles) step(A0, B0, A2, B2, t);
    if (t + 1 < ktiles) mma_tile<BMODE>(acc, A1, B1, wm, brow, lane);
    wait_vmem();
  } else if constexpr (!REG_B) {
    // bf16 B: 32 KiB A and B tiles.  The weights (B) stream from HBM, so they
    // get a three-stage ring and the activations (A, L2 resident in the
    // MLP / projection shapes) two stages: 2 x 32 + 3 x 32 = 160 KiB, all of
    // the CU's LDS.  Per tile t: A(t + 1) is issued first, then B(t + 2);
    // the closing vmcnt leaves only B(t + 2) in flight, so A(t + 1) and
    // B(t + 1) (issued a tile earlier) have landed.  The loop is unrolled
    // six ways so every stage address is static.
    __shared__ __attribute__((aligned(1024))) uint8_t A0[BM * 128];
    __shared__ __attribute__((aligned(1024))) uint8_t A1[BM * 128];
    __shared__ __attribute__((aligned(1024))) uint8_t B0[BN * BROW];
    __shared__ __attribute__((aligned(1024))) uint8_t B1[BN * BROW];
    __shared__ __attribute__((aligned(1024))) uint8_t B2[BN * BROW];
    issue_a(A0, 0);
    issue_b(B0, 0);
    issue_b(B1, BK);
    wait_vmem_but<NVB>();
    barrier_no_fence();
    auto step = [&](uint8_t *Ac, uint8_t *Bc, uint8_t *An, uint8_t *Bn, int tt) __attribute__((always_inline)) {
      issue_a(An, (int64_t)(tt + 1) * BK);
      issue_b(Bn, (int64_t)(tt + 2) * BK);
      mma_tile<BMODE>(acc, Ac, Bc, wm, brow, lane);
      schedule_ktile<NDS, NVM>();
      wait_vmem_but<NVB>();
      barrier_no_fence();
    };
    // tile t: A in A[t % 2], B in B[t % 3]; step writes A[(t+1) % 2], B[(t+2) % 3]
    int t = 0;
    for (; t + 6 <= ktiles; t += 6) {
      step(A0, B0, A1, B2, t);
      step(A1, B1, A0, B0, t + 1);
      step(A0, B2, A1, B1, t + 2);
      step(A1, B0, A0, B2, t + 3);
      step(A0, B1, A1, B0, t + 4);
      step(A1, B2, A0, B1, t + 5);
    }
    // remaining 0..5 tiles, same rotation
    if (t < ktiles) step(A0, B0, A1, B2, t);
    if (t + 1 < ktiles) step(A1, B1, A0, B0, t + 1);
    if (t + 2 < ktiles) step(A0, B2, A1, B1, t + 2);
    if (t + 3 < ktiles) step(A1, B0, A0, B2, t + 3);
    if (t + 4 < ktiles) step(A0, B1, A1, B0, t + 4);
    wait_vmem();
  } else {
    // fp8 NN weights go through registers (transposed there): two stages
    __shared__ __attribute__((aligned(1024))) uint8_t A0[BM * 128];
    __shared__ __attribute__((aligned(1024))) uint8_t A1[BM * 128];
    __shared__ __attribute__((aligned(1024))) uint8_t B0[BN * BROW];
    __shared__ __attribute__((aligned(1024))) uint8_t B1[BN * BROW];
    issue(A0, B0, 0);
    wait_vmem();
    store_nn(sn, B0);
    wait_vmem();
    __syncthreads();
    int t = 0;
    for (; t + 2 <= ktiles; t += 2) {
      issue(A1, B1, (int64_t)(t + 1) * BK);
      mma_tile<BMODE>(acc, A0, B0, wm, brow, lane);
      schedule_ktile<NDS, NVM>();
      wait_vmem();
      store_nn(sn, B1);
      wait_vmem();
      __syncthreads();
      // past the last tile this reads zeros (K offset out of range) into the idle stage
      issue(A0, B0, (int64_t)(t + 2) * BK);
      mma_tile<BMODE>(acc, A1, B1, wm, brow, lane);
      schedule_ktile<NDS, NVM>();
      if (t + 2 < ktiles) {
        wait_vmem();
        store_nn(sn, B0);
      }
      wait_vmem();
      __syncthreads();
    }
    if (t < ktiles) mma_tile<BMODE>(acc, A0, B0, wm, brow, lane);
  }

  // epilogue.  The MFMAs computed C^T tiles (B fragment as the A operand),
  // so a lane holds row m = m0 + wm*128 + i*32 + l32 of C and, per tile,
  // 16 columns n = (tile column) + 8 q + 4 lhi + e (q, e = 0..3): runs of 4
  // consecutive columns, stored / read as one vector.
  const int l32 = lane & 31, lhi = lane >> 5;
  const bool vec = (a.flags & GEMM_VEC) != 0;
  auto put4 = [&](int64_t row, int64_t col, const float (&v)[4]) {
    if (vec && col + 3 < a.N) {
      OutT<TC>::store4(a.C, row * a.ldc + col, v);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (col + e < a.N) OutT<TC>::store(a.C, row * a.ldc + col + e, v[e]);
    }
  };
  if (SWIGLU) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t nb = n0 + wn * 64 + j * 32 + lhi * 4;
      float sg[16], su[16];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t col = nb + q * 8 + e;
          const bool in = (a.flags & GEMM_SCALE) && col < a.N;
          sg[q * 4 + e] = in ? a.scale0[col] : 1.f;
          su[q * 4 + e] = in ? a.scale1[col] : 1.f;
        }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t row = m0 + wm * 128 + i * 32 + l32;
        if (row >= a.M) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t col = nb + q * 8;
          if (col >= a.N) continue;
          float h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float g = acc[i][j][q * 4 + e] * sg[q * 4 + e];
            const float u = acc[i][j + 2][q * 4 + e] * su[q * 4 + e];
            // silu(g) = g / (1 + exp(-g)) from the hardware 2^x and
            // reciprocal (about 2 ulp in fp32, far below the bf16 output
            // rounding); the accurate expf / division sequences would keep
            // the MFMA pipe idle for ~10% of a K = 4096 tile
            const float ex = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
            h[e] = g * __builtin_amdgcn_rcpf(1.0f + ex) * u;
          }
          put4(row, col, h);
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t nb = n0 + wn * 128 + j * 32 + lhi * 4;
      float sc[16], bi[16];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t col = nb + q * 8 + e;
          sc[q * 4 + e] = ((a.flags & GEMM_SCALE) && col < a.N) ? a.scale0[col] : 1.f;
          bi[q * 4 + e] = ((a.flags & GEMM_BIAS) && col < a.N)
                              ? bf16_to_f32(reinterpret_cast<const uint16_t *>(a.bias)[col]) : 0.f;
        }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t row = m0 + wm * 128 + i * 32 + l32;
        if (row >= a.M) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t col = nb + q * 8;
          if (col >= a.N) continue;
          float r4[4] = {0.f, 0.f, 0.f, 0.f};
          if (a.flags & GEMM_RESID) {
            if (vec && col + 3 < a.N) {
              OutT<TC>::load4(a.resid, row * a.ldc + col, r4);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (col + e < a.N) r4[e] = OutT<TC>::load(a.resid, row * a.ldc + col + e);
            }
          }
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[i][j][q * 4 + e] * sc[q * 4 + e] + bi[q * 4 + e] + r4[e];
          put4(row, col, v);
        }
      }
    }
  }
}

#define NK_GEMM(NT, FP8, SW, TC, name)                                                   \
  extern "C" __global__ __launch_bounds__(NTHREADS, 1) void name(GemmArgs a) {           \
    gemm_body<NT, FP8, SW, TC>(a);                                                       \
  }

NK_GEMM(false, false, false, bf16, nk_gemm_nn_bf16_bf16)
NK_GEMM(false, false, false, float, nk_gemm_nn_bf16_f32)
NK_GEMM(true, false, false, bf16, nk_gemm_nt_bf16_bf16)
NK_GEMM(true, false, false, float, nk_gemm_nt_bf16_f32)
NK_GEMM(false, false, true, bf16, nk_gemm_swiglu_nn_bf16_bf16)
NK_GEMM(true, false, true, bf16, nk_gemm_swiglu_nt_bf16_bf16)
NK_GEMM(true, true, false, bf16, nk_gemm_nt_e4m3_bf16)
NK_GEMM(true, true, false, float, nk_gemm_nt_e4m3_f32)
NK_GEMM(true, true, true, bf16, nk_gemm_swiglu_nt_e4m3_bf16)
NK_GEMM(false, true, false, bf16, nk_gemm_nn_e4m3_bf16)
