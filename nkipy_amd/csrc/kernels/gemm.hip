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
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

#define BM 256
#define BN 256
#define BK 64
#define NTHREADS 256
// Tile rows per group of the XCD-local walk.  Measured on MI355X (us, 8-wave
// kernel, GROUP_M 1 / 2 / 4 / 8): NT bf16 16384x6144x4096 731 / 709 / 685 /
// 771, NT fp8 same shape 692 / 694 / 668 / 730, NN 4096x4096x14336 353 /
// 352 / 351 / 358, fp8 SwiGLU 16384x14336x4096 unchanged.
#define GROUP_M 4

enum {
  GEMM_BIAS = 1,      // + bias[col] (bf16)
  GEMM_SCALE = 2,     // * scale[col] (fp32), per output column (fp8 weights)
  GEMM_RESID = 4,     // + residual[row][col] (same dtype as C)
  GEMM_VEC = 8,       // C / residual rows allow aligned 4-element vector access
  GEMM_RND_BIAS = 16, // round the (scaled) product to bf16 before the bias add
  GEMM_RND_RESID = 32,// round to bf16 before the residual add
  GEMM_ROWS16 = 64,   // bf16 C / residual rows take aligned 16-byte chunks (N, ldc
                      // multiples of 8) and a residual is added to a rounded value:
                      // the 8-wave kernels may stage the output tile through LDS
};
// The rounding flags keep the cast points of the traced NumPy code: e.g.
// ``z + (x @ w).astype(bf16)`` rounds the product before the add.

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
  int32_t flags;
  int32_t group_m;     // tile rows per group of the tile walk; 0: GROUP_M
  // rotary embedding of the q / k columns (the *_rope kernels only)
  const float *rope_cos;  // fp32 [position][64], row stride rope_ts
  const float *rope_sin;
  void *rope_q;           // M x rope_nq bf16: rotated columns 0 .. rope_nq-1
  void *rope_k;           // M x rope_nk bf16: rotated columns rope_nq ..
  int64_t rope_ts;
  int32_t rope_seq;       // row m sits at position m % rope_seq
  int32_t rope_nq, rope_nk, rope_pad;
  // split-K entries (*_splitk): K ranges of kc (a multiple of 64), range
  // blockIdx.y; fp32 partial sums of range s at C + s * M * ldc
  int32_t ksplit, kc;
};

// ---------------------------------------------------------------------------
// element helpers
// ---------------------------------------------------------------------------
// fp8 -> bf16 staging uses nk::e4m3x8_to_bf16x8 (common.h)

// (product + bias) + residual with the optional bf16 roundings in between
__device__ __forceinline__ float epilogue(int flags, float prod, float bias, float resid) {
  if (flags & GEMM_RND_BIAS) prod = bf16_to_f32(f32_to_bf16(prod));
  float v = prod + bias;
  if (flags & GEMM_RND_RESID) v = bf16_to_f32(f32_to_bf16(v));
  return v + resid;
}

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
        make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
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
// chunks stored at chunk ^ swz(row).  With NW waves, wave w moves blocks
// b = NW j + w of 8 rows; lane l fills stored slot (row, l % 8), so it fetches
// logical chunk (l % 8) ^ swz(row) -- the same chunk for every j, since
// swz(row) only depends on (4 b + l / 16) mod 8 and b = w mod 2.
template <int NW>
__device__ __forceinline__ DmaPlan<32 / NW> plan_rows_bf16(bool split, int64_t r_first, int64_t nrows, int64_t ld,
                                                           int wave, int lane) {
  DmaPlan<32 / NW> p;
  const int lc = (lane & 7) ^ swz(wave * 8 + (lane >> 3), 0);  // row of move j = 0
  p.kofs = lc * 8;
#pragma unroll
  for (int j = 0; j < 32 / NW; ++j) {
    const int b = j * NW + wave;
    const int row = b * 8 + (lane >> 3);
    const int64_t rr = r_first + ((split && b >= 16) ? row - 128 : row);
    p.base[j] = rr < nrows ? (uint32_t)((rr * ld + p.kofs) * 2) : OOB;
  }
  return p;
}

template <int NW>
__device__ __forceinline__ void dma_rows_bf16(const DmaPlan<32 / NW> &p, __amdgpu_buffer_rsrc_t r0,
                                              __amdgpu_buffer_rsrc_t r1, bool split, uint8_t *S, int64_t k0,
                                              int64_t K, int wave) {
#pragma unroll
  for (int j = 0; j < 32 / NW; ++j) {
    const int b = j * NW + wave;
    dma16((split && b >= 16) ? r1 : r0, S + b * 1024, dma_off(p.base[j], k0, p.kofs, K, 2));
  }
}

// fp8 B^T tile (NT weights): 256 rows x 64 codes = 64-byte rows, 16-byte
// chunks stored at chunk ^ ((row >> 2) & 3).  Blocks of 16 rows.
__device__ __forceinline__ int swz8(int row) { return (row >> 2) & 3; }

template <int NW>
__device__ __forceinline__ DmaPlan<16 / NW> plan_rows_fp8(bool split, int64_t r_first, int64_t nrows, int64_t ld,
                                                          int wave, int lane) {
  DmaPlan<16 / NW> p;
  const int lc = (lane & 3) ^ swz8(wave * 16 + (lane >> 2));  // row of move j = 0
  p.kofs = lc * 16;
#pragma unroll
  for (int j = 0; j < 16 / NW; ++j) {
    const int b = j * NW + wave;
    const int row = b * 16 + (lane >> 2);
    const int64_t rr = r_first + ((split && b >= 8) ? row - 128 : row);
    p.base[j] = rr < nrows ? (uint32_t)(rr * ld + p.kofs) : OOB;
  }
  return p;
}

template <int NW>
__device__ __forceinline__ void dma_rows_fp8(const DmaPlan<16 / NW> &p, __amdgpu_buffer_rsrc_t r0,
                                             __amdgpu_buffer_rsrc_t r1, bool split, uint8_t *S, int64_t k0,
                                             int64_t K, int wave) {
#pragma unroll
  for (int j = 0; j < 16 / NW; ++j) {
    const int b = j * NW + wave;
    dma16((split && b >= 8) ? r1 : r0, S + b * 1024, dma_off(p.base[j], k0, p.kofs, K, 1));
  }
}

// bf16 NN B tile (K x N weights, N contiguous): stored as two column halves
// [64 k][128 n] with 256-byte rows (half 0 = tile columns 0..127, half 1 =
// 128..255; in SwiGLU mode gate and up), 16-byte chunks at chunk ^ nnswz(k).
// MFMA fragments are read with ds_read_b64_tr_b16 (below).  Blocks of 4 rows;
// block b = NW j + w covers k rows (b mod 16) * 4 + l / 16 of half b / 16.
__device__ __forceinline__ int nnswz(int k) { return (k & 3) << 2; }

template <int NW>
__device__ __forceinline__ int nn_krow(int j, int wave, int lane) { return ((j * NW + wave) & 15) * 4 + (lane >> 4); }

template <int NW>
__device__ __forceinline__ DmaPlan<32 / NW> plan_nn_bf16(bool split, int64_t n0, int64_t N, int64_t ld, int wave,
                                                         int lane) {
  DmaPlan<32 / NW> p;
  p.kofs = 0;
#pragma unroll
  for (int j = 0; j < 32 / NW; ++j) {
    const int b = j * NW + wave;
    const int half = b >> 4;
    const int k = nn_krow<NW>(j, wave, lane);
    const int lc = (lane & 15) ^ nnswz(k);
    const int64_t col = n0 + (split ? 0 : half * 128) + lc * 8;
    p.base[j] = col < N ? (uint32_t)((k * ld + col) * 2) : OOB;
  }
  return p;
}

template <int NW>
__device__ __forceinline__ void dma_nn_bf16(const DmaPlan<32 / NW> &p, __amdgpu_buffer_rsrc_t r0,
                                            __amdgpu_buffer_rsrc_t r1, bool split, uint8_t *S, int64_t k0,
                                            int64_t K, int64_t ld, int wave, int lane) {
#pragma unroll
  for (int j = 0; j < 32 / NW; ++j) {
    const int b = j * NW + wave;
    dma16((split && (b >> 4)) ? r1 : r0, S + b * 1024,
          dma_off(p.base[j], k0, nn_krow<NW>(j, wave, lane), K, ld * 2));
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

// Fragments of k16 step kk: NA A tiles (rows arow0 + 32 i ..) and the four
// B tiles of brow.
template <int BM_, int NA>
__device__ __forceinline__ void read_frags(bf16x8_t (&af)[NA], bf16x8_t (&bf)[4], const uint8_t *As,
                                           const uint8_t *Bs, int kk, int arow0, const int (&brow)[4],
                                           int lane) {
  const int l32 = lane & 31, lhi = lane >> 5;
  const int chunk = kk * 2 + lhi;
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int row = arow0 + i * 32 + l32;
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
  read_frags<BM_, 4>(af[0], bf[0], As, Bs, 0, wm * 128, brow, lane);
#pragma unroll
  for (int kk = 0; kk < BK / 16; ++kk) {
    if (kk + 1 < BK / 16)
      read_frags<BM_, 4>(af[(kk + 1) & 1], bf[(kk + 1) & 1], As, Bs, kk + 1, wm * 128, brow, lane);
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

// Epilogue.  The MFMAs computed C^T tiles (B fragment as the A operand), so
// a lane holds row rbase + 32 i + l32 of C and, per tile, 16 columns
// n = (tile column) + 8 q + 4 lhi + e (q, e = 0..3): runs of 4 consecutive
// columns, stored / read as one vector.
template <bool SWIGLU, typename TC, int NA>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs &a, const f32x16 (&acc)[NA][4], int64_t rbase,
                                              int64_t n0, int wn, int lane) {
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
      for (int i = 0; i < NA; ++i) {
        const int64_t row = rbase + i * 32 + l32;
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
      for (int i = 0; i < NA; ++i) {
        const int64_t row = rbase + i * 32 + l32;
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
          for (int e = 0; e < 4; ++e) v[e] = epilogue(a.flags, acc[i][j][q * 4 + e] * sc[q * 4 + e],
                                                      bi[q * 4 + e], r4[e]);
          put4(row, col, v);
        }
      }
    }
  }
}

// Output tile of this workgroup, XCD aware: consecutive workgroup ids are
// dealt to the 8 XCDs round robin, so ids are remapped so that each XCD
// receives a contiguous run of tiles, walked in groups of GROUP_M tile rows.
__device__ __forceinline__ void gemm_tile(const GemmArgs &a, int &tm, int &tn) {
  const int ntiles = a.tiles_m * a.tiles_n;
  int pid = blockIdx.x;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  const int gm = a.group_m > 0 ? a.group_m : GROUP_M;
  const int in_group = gm * a.tiles_n;
  const int group = pid / in_group;
  const int first_m = group * gm;
  const int gsize = min(a.tiles_m - first_m, gm);
  tm = first_m + (pid % in_group) % gsize;
  tn = (pid % in_group) / gsize;
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

  int tm, tn;
  gemm_tile(a, tm, tn);
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
  const DmaPlan<8> pa = plan_rows_bf16<4>(false, m0, a.M, a.lda, wave, lane);
  DmaPlan<8> pb16;
  DmaPlan<4> pb8;
  if (NT && FP8) pb8 = plan_rows_fp8<4>(SWIGLU, n0, a.N, a.ldb, wave, lane);
  if (NT && !FP8) pb16 = plan_rows_bf16<4>(SWIGLU, n0, a.N, a.ldb, wave, lane);
  if (!NT && !FP8) pb16 = plan_nn_bf16<4>(SWIGLU, n0, a.N, a.ldb, wave, lane);
  auto issue_a = [&](uint8_t *As, int64_t k0) { dma_rows_bf16<4>(pa, ra, ra, false, As, k0, a.K, wave); };
  auto issue_b = [&](uint8_t *Bs, int64_t k0) {
    if (NT) {
      if (FP8)
        dma_rows_fp8<4>(pb8, rb0, rb1, SWIGLU, Bs, k0, a.K, wave);
      else
        dma_rows_bf16<4>(pb16, rb0, rb1, SWIGLU, Bs, k0, a.K, wave);
    } else if (REG_B) {
      load_nn<FP8, SWIGLU>(sn, a, rb0, rb1, n0, k0);
    } else {
      dma_nn_bf16<4>(pb16, rb0, rb1, SWIGLU, Bs, k0, a.K, a.ldb, wave, lane);
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

  gemm_epilogue<SWIGLU, TC, 4>(a, acc, m0 + wm * 128, n0, wn, lane);
}

template <int N> struct Int {
  static constexpr int value = N;
};

// ---------------------------------------------------------------------------
// 8-wave ping-pong kernel (NT weights, and bf16 NN weights; the default)
// ---------------------------------------------------------------------------
// Same 256 x 256 output tiles, 512 threads: wave w sits on SIMD w % 4, so each
// SIMD hosts one wave of group 0 (waves 0..3, output rows 0..127 of the
// tile) and one of group 1 (waves 4..7, rows 128..255); each wave owns 64
// rows x 128 B^T rows (4 x 8 tiles of v_mfma_f32_16x16x32_bf16, which
// sustains a higher rate than the 32x32x16 form on random operands; 128
// accumulators).  K advances in phases of 32 (one MFMA k step); phase p is
// computed by group 0 in slot 2p and by group 1 in slot 2p + 1, slots being
// separated by workgroup barriers, and each group reads (and, for fp8,
// decodes) a phase's fragments from LDS into registers in the slot before it
// computes it:
//   slot 2p:     group 0 computes phase p,  group 1 loads phase p
//   slot 2p + 1: group 1 computes phase p,  group 0 loads phase p + 1
// so the matrix pipe of a SIMD is fed alternately by its two waves and the
// barrier of one slot is covered by the MFMAs the other wave has queued.
// LDS holds a ring of R half-tile stages (A 256 x 32 bf16, B 256 x 32 bf16
// or fp8): the stage of phase p is free once slot 2p ends, so in slot 2p + 1
// the DMAs of phase p + R go into it; before the barrier that closes slot 2p
// each wave waits until its DMAs of phase p + 1 have landed (all but the
// R - 2 newest phases), which leaves 2R - 2 slots for a DMA to arrive.  The
// DMAs are issued from inline asm: the compiler does not track them, so it
// adds no waits of its own (its tracking of LDS DMA targets is lost across
// the loop's back edge, and its waits then drain the whole ring); every
// ordering is the explicit vmcnt / lgkmcnt / barrier above.
//
// Half-tile layouts (16-byte chunks XOR-swizzled by row, conflict-free for
// the fragment reads below):
//   A, bf16 B^T: 256 rows x 64 bytes, chunk c (k 8c..8c+7) at c ^ hswz(row)
//   fp8 B^T:     256 rows x 32 bytes, chunk c (k 16c..) at c ^ hswz8(row)
//   NN bf16 B:   [2 column halves][32 k][256 bytes], chunk at c ^ nnswz(k)
__device__ __forceinline__ int hswz(int row) { return (row >> 2) & 3; }
__device__ __forceinline__ int hswz8(int row) { return (row >> 3) & 1; }

// Epilogue of the 16x16 tiles of the 8-wave kernel: lane (g, i) holds, per
// tile (i', j), output row rbase + 16 i' + i and the 4 consecutive columns
// cbase + 16 j + 4 g + 0..3 (SwiGLU: tiles j < 4 gate and j + 4 up of the
// same output columns cbase + 16 j + ..).
// Loads are issued ahead of the stores: the residual of tile column j + 1 is
// fetched before column j is stored (the compiler may not move a load past a
// store that can alias it, and C may be the residual buffer itself -- each
// lane reads only the elements it writes, so the early reads are exact).
template <bool SWIGLU, typename TC, int NI>
__device__ __forceinline__ void gemm_epilogue16(const GemmArgs &a, const f32x4 (&acc)[NI][8], int64_t rbase,
                                                int64_t cbase, int lane) {
  const int l16 = lane & 15, g4 = lane >> 4;
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
  constexpr int NJ = SWIGLU ? 4 : 8;
  // per-column factors of every tile column, fetched up front
  float sc[NJ][4], su[NJ][4], bi[NJ][4];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int64_t col = cbase + 16 * j + 4 * g4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool in = col + e < a.N;
      sc[j][e] = ((a.flags & GEMM_SCALE) && in) ? a.scale0[col + e] : 1.f;
      su[j][e] = (SWIGLU && (a.flags & GEMM_SCALE) && in) ? a.scale1[col + e] : 1.f;
      bi[j][e] = (!SWIGLU && (a.flags & GEMM_BIAS) && in)
                     ? bf16_to_f32(reinterpret_cast<const uint16_t *>(a.bias)[col + e]) : 0.f;
    }
  }
  if constexpr (SWIGLU) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int64_t col = cbase + 16 * j + 4 * g4;
      if (col >= a.N) continue;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int64_t row = rbase + 16 * i + l16;
        if (row >= a.M) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float g = acc[i][j][e] * sc[j][e];
          const float u = acc[i][j + 4][e] * su[j][e];
          // silu(g) = g / (1 + exp(-g)) from the hardware 2^x and reciprocal
          const float ex = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
          v[e] = g * __builtin_amdgcn_rcpf(1.0f + ex) * u;
        }
        put4(row, col, v);
      }
    }
  } else {
    const bool res = (a.flags & GEMM_RESID) != 0;
    // residual of tile column j, rows i: 4 elements each
    auto fetch = [&](int j, float (&r)[NI][4]) {
      const int64_t col = cbase + 16 * j + 4 * g4;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int64_t row = rbase + 16 * i + l16;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[i][e] = 0.f;
        if (!res || row >= a.M || col >= a.N) continue;
        if (vec && col + 3 < a.N) {
          OutT<TC>::load4(a.resid, row * a.ldc + col, r[i]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (col + e < a.N) r[i][e] = OutT<TC>::load(a.resid, row * a.ldc + col + e);
        }
      }
    };
    float rc[NI][4], rn[NI][4];
    fetch(0, rc);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (j + 1 < NJ) fetch(j + 1, rn);
      const int64_t col = cbase + 16 * j + 4 * g4;
      if (col < a.N) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const int64_t row = rbase + 16 * i + l16;
          if (row >= a.M) continue;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = epilogue(a.flags, acc[i][j][e] * sc[j][e], bi[j][e], rc[i][e]);
          put4(row, col, v);
        }
      }
      if (j + 1 < NJ) {
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) rc[i][e] = rn[i][e];
      }
    }
  }
}

// Epilogue through LDS (bf16 C, flag GEMM_ROWS16, the LDS ring idle): each
// wave writes its converted values (scale, bias, SwiGLU; with a residual,
// the value rounded to bf16 before the add, which is what is stored) into a
// row-major tile T of 256 rows (padded by 16 bytes against bank conflicts);
// then all 512 threads walk T in 16-byte chunks along the rows, add the
// residual and store, so every global access covers whole cache lines
// (the per-lane 8-byte stores of gemm_epilogue16 cover 32-byte row pieces,
// four times as many requests).  Same arithmetic as gemm_epilogue16.
typedef __attribute__((address_space(3))) uint8_t lds_b;
typedef unsigned lds_u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned lds_u32x4_t __attribute__((ext_vector_type(4)));
// 8-byte store / 16-byte load through an LDS-typed pointer (ds_write_b64 /
// ds_read_b128 rather than the flat forms a generic pointer would give)
__device__ __forceinline__ void lds_st8(lds_b *p, uint32_t lo, uint32_t hi) {
  lds_u32x2_t v;
  v.x = lo;
  v.y = hi;
  *reinterpret_cast<__attribute__((address_space(3))) lds_u32x2_t *>(p) = v;
}
__device__ __forceinline__ uint4 lds_ld16(const lds_b *p) {
  const lds_u32x4_t v = *reinterpret_cast<const __attribute__((address_space(3))) lds_u32x4_t *>(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

template <bool SWIGLU, int NI>
__device__ __forceinline__ void gemm_epilogue_lds(const GemmArgs &a, const f32x4 (&acc)[NI][8], int64_t m0,
                                                  int64_t n0, int arow0, int bw0, int lane, uint8_t *T) {
  constexpr int OC = SWIGLU ? 128 : 256;  // output columns of the tile
  constexpr int TS = OC * 2 + 16;         // T row stride in bytes
  constexpr int NJ = SWIGLU ? 4 : 8;
  const int l16 = lane & 15, g4 = lane >> 4;
  // this lane's first T element (row arow0 + l16, column bw0 + 4 g4); tile
  // (i, j) is at + i * 16 rows + j * 16 columns, immediates off one base
  // (an LDS-typed pointer, so the accesses are ds_* and not flat)
  lds_b *const TL = (lds_b *)T;
  lds_b *tb = TL + (arow0 + l16) * TS + (bw0 + 4 * g4) * 2;
  asm volatile("" : "+v"(tb));
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int ct = bw0 + 16 * j + 4 * g4;
    const int64_t col = n0 + ct;
    float sc[4], su[4], bi[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool in = col + e < a.N;
      sc[e] = ((a.flags & GEMM_SCALE) && in) ? a.scale0[col + e] : 1.f;
      su[e] = (SWIGLU && (a.flags & GEMM_SCALE) && in) ? a.scale1[col + e] : 1.f;
      bi[e] = (!SWIGLU && (a.flags & GEMM_BIAS) && in)
                  ? bf16_to_f32(reinterpret_cast<const uint16_t *>(a.bias)[col + e]) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (SWIGLU) {
          const float g = acc[i][j][e] * sc[e];
          const float u = acc[i][j + 4][e] * su[e];
          const float ex = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
          v[e] = g * __builtin_amdgcn_rcpf(1.0f + ex) * u;
        } else {
          float prod = acc[i][j][e] * sc[e];
          if (a.flags & GEMM_RND_BIAS) prod = bf16_to_f32(f32_to_bf16(prod));
          v[e] = prod + bi[e];
        }
      }
      lds_st8(tb + 16 * i * TS + 32 * j, pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    }
  }
  barrier_no_fence();
  // every read (the tile's chunks from LDS, the residual's from memory) is
  // issued before the first store: a store may alias the residual (C may be
  // the residual buffer), so reads interleaved with the stores would each
  // wait a full memory latency.  Each thread reads only the residual chunks
  // it writes, so reading them all first is exact.
  constexpr int CPR = OC / 8;           // 16-byte chunks per row
  constexpr int NIT = 256 * CPR / 512;  // chunks per thread
  const bool res = (a.flags & GEMM_RESID) != 0;
  uint4 w[NIT], r[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int k = threadIdx.x + 512 * it;
    const int rt = k / CPR, ch = k % CPR;
    const int64_t row = m0 + rt, col = n0 + ch * 8;
    w[it] = lds_ld16(TL + rt * TS + ch * 16);
    r[it] = make_uint4(0, 0, 0, 0);
    if (res && row < a.M && col < a.N)
      r[it] = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(a.resid) + row * a.ldc + col);
  }
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int k = threadIdx.x + 512 * it;
    const int rt = k / CPR, ch = k % CPR;
    const int64_t row = m0 + rt, col = n0 + ch * 8;
    if (row >= a.M || col >= a.N) continue;
    uint4 v = w[it];
    if (res) {
      const uint32_t wv[4] = {v.x, v.y, v.z, v.w}, rv[4] = {r[it].x, r[it].y, r[it].z, r[it].w};
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float lo = __uint_as_float(wv[q] << 16) + __uint_as_float(rv[q] << 16);
        const float hi = __uint_as_float(wv[q] & 0xffff0000u) + __uint_as_float(rv[q] & 0xffff0000u);
        o[q] = pack_bf16x2(lo, hi);
      }
      v = make_uint4(o[0], o[1], o[2], o[3]);
    }
    *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(a.C) + row * a.ldc + col) = v;
  }
}

// Epilogue of the rotary-embedding kernels: columns below rope_nq + rope_nk
// are heads of 128 (q heads, then k heads), and a wave's 128 columns are one
// head (cbase is a multiple of 128), so lane (g, i) holds frequency
// 16 j + 4 g + e of both halves: x0 in tile j, x1 in tile j + 4.  Per element,
// as the traced NumPy code evaluates it:
//   x0, x1 = bf16(product * scale)                     (the projection's cast)
//   out0 = bf16(x0 * cos - x1 * sin), out1 = bf16(x0 * sin + x1 * cos)
// with every product and sum rounded to fp32 separately (no fused
// multiply-add).  The rotated head goes to rope_q / rope_k; C keeps only the
// remaining (value) columns.
template <int NI>
__device__ __forceinline__ void gemm_epilogue_rope(const GemmArgs &a, const f32x4 (&acc)[NI][8], int64_t rbase,
                                                   int64_t cbase, int lane) {
  const int l16 = lane & 15, g4 = lane >> 4;
  const bool isq = cbase < a.rope_nq;
  uint16_t *dst = reinterpret_cast<uint16_t *>(isq ? a.rope_q : a.rope_k);
  const int64_t ldd = isq ? a.rope_nq : a.rope_nk;
  const int64_t c0 = isq ? cbase : cbase - a.rope_nq;
  const bool scaled = (a.flags & GEMM_SCALE) != 0;
  // table row offsets of the lane's rows (rows past M read row 0: in bounds, unused)
  int64_t toff[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int64_t row = rbase + 16 * i + l16;
    toff[i] = (row < a.M ? (int64_t)((int32_t)row % a.rope_seq) : 0) * a.rope_ts + 4 * g4;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int d = 16 * j + 4 * g4;
    // one batch of loads per tile column: its scales and the 2 x NI table vectors
    float s0[4], s1[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s0[e] = scaled ? a.scale0[cbase + d + e] : 1.f;
      s1[e] = scaled ? a.scale0[cbase + 64 + d + e] : 1.f;
    }
    float4 c[NI], s[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      c[i] = *reinterpret_cast<const float4 *>(a.rope_cos + toff[i] + 16 * j);
      s[i] = *reinterpret_cast<const float4 *>(a.rope_sin + toff[i] + 16 * j);
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int64_t row = rbase + 16 * i + l16;
      if (row >= a.M) continue;
      const float cv[4] = {c[i].x, c[i].y, c[i].z, c[i].w}, sv[4] = {s[i].x, s[i].y, s[i].z, s[i].w};
      float y0[4], y1[4];
      {
#pragma clang fp contract(off)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x0 = bf16_to_f32(f32_to_bf16(acc[i][j][e] * s0[e]));
          const float x1 = bf16_to_f32(f32_to_bf16(acc[i][j + 4][e] * s1[e]));
          y0[e] = x0 * cv[e] - x1 * sv[e];
          y1[e] = x0 * sv[e] + x1 * cv[e];
        }
      }
      OutT<bf16>::store4(dst, row * ldd + c0 + d, y0);
      OutT<bf16>::store4(dst, row * ldd + c0 + 64 + d, y1);
    }
  }
}

// The rotary epilogue staged through LDS (the ring idle): each wave writes
// its head -- rotated as in gemm_epilogue_rope for q / k heads, the scaled
// projection for value columns -- as bf16 into a row-major tile T (256 rows,
// padded by 16 bytes), then all 512 threads move 16-byte row chunks to
// rope_q, rope_k or C by column, so every global store covers whole lines.
// Same arithmetic as gemm_epilogue_rope / gemm_epilogue16.
template <int NI>
__device__ __forceinline__ void gemm_epilogue_rope_lds(const GemmArgs &a, const f32x4 (&acc)[NI][8], int64_t m0,
                                                       int64_t n0, int arow0, int bw0, int lane, uint8_t *T) {
  constexpr int TS = 256 * 2 + 16;  // T row stride in bytes
  const int l16 = lane & 15, g4 = lane >> 4;
  lds_b *const TL = (lds_b *)T;  // ds_* accesses, not flat
  lds_b *tb = TL + (arow0 + l16) * TS + (bw0 + 4 * g4) * 2;
  asm volatile("" : "+v"(tb));
  const int64_t cbase = n0 + bw0;  // this wave's 128 columns: one head
  const bool scaled = (a.flags & GEMM_SCALE) != 0;
  if (cbase < (int64_t)a.rope_nq + a.rope_nk) {
    int64_t toff[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int64_t row = m0 + arow0 + 16 * i + l16;
      toff[i] = (row < a.M ? (int64_t)((int32_t)row % a.rope_seq) : 0) * a.rope_ts + 4 * g4;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 16 * j + 4 * g4;
      float s0[4], s1[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s0[e] = scaled ? a.scale0[cbase + d + e] : 1.f;
        s1[e] = scaled ? a.scale0[cbase + 64 + d + e] : 1.f;
      }
      float4 c[NI], sn[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        c[i] = *reinterpret_cast<const float4 *>(a.rope_cos + toff[i] + 16 * j);
        sn[i] = *reinterpret_cast<const float4 *>(a.rope_sin + toff[i] + 16 * j);
      }
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const float cv[4] = {c[i].x, c[i].y, c[i].z, c[i].w}, sv[4] = {sn[i].x, sn[i].y, sn[i].z, sn[i].w};
        float y0[4], y1[4];
        {
#pragma clang fp contract(off)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x0 = bf16_to_f32(f32_to_bf16(acc[i][j][e] * s0[e]));
            const float x1 = bf16_to_f32(f32_to_bf16(acc[i][j + 4][e] * s1[e]));
            y0[e] = x0 * cv[e] - x1 * sv[e];
            y1[e] = x0 * sv[e] + x1 * cv[e];
          }
        }
        lds_st8(tb + 16 * i * TS + 32 * j, pack_bf16x2(y0[0], y0[1]), pack_bf16x2(y0[2], y0[3]));
        lds_st8(tb + 16 * i * TS + 32 * (j + 4), pack_bf16x2(y1[0], y1[1]), pack_bf16x2(y1[2], y1[3]));
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t col = cbase + 16 * j + 4 * g4;
      float sc[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[e] = (scaled && col + e < a.N) ? a.scale0[col + e] : 1.f;
#pragma unroll
      for (int i = 0; i < NI; ++i)
        lds_st8(tb + 16 * i * TS + 32 * j, pack_bf16x2(acc[i][j][0] * sc[0], acc[i][j][1] * sc[1]),
                pack_bf16x2(acc[i][j][2] * sc[2], acc[i][j][3] * sc[3]));
    }
  }
  barrier_no_fence();
  constexpr int CPR = 32;               // 16-byte chunks per tile row
  constexpr int NIT = 256 * CPR / 512;  // chunks per thread
  const int64_t nrot = (int64_t)a.rope_nq + a.rope_nk;
  uint4 wt[NIT];  // every LDS read issued before the first store
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int k = threadIdx.x + 512 * it;
    wt[it] = lds_ld16(TL + (k / CPR) * TS + (k % CPR) * 16);
  }
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int k = threadIdx.x + 512 * it;
    const int rt = k / CPR, ch = k % CPR;
    const int64_t row = m0 + rt, col = n0 + ch * 8;
    if (row >= a.M || col >= a.N) continue;
    const uint4 w = wt[it];
    uint16_t *dst = col < a.rope_nq ? reinterpret_cast<uint16_t *>(a.rope_q) + row * a.rope_nq + col
                    : col < nrot   ? reinterpret_cast<uint16_t *>(a.rope_k) + row * a.rope_nk + (col - a.rope_nq)
                                   : reinterpret_cast<uint16_t *>(a.C) + row * a.ldc + col;
    *reinterpret_cast<uint4 *>(dst) = w;
  }
}

// LDS DMA as in dma16_asm, with a uniform (SGPR) part of the offset: voff + soff
__device__ __forceinline__ void dma16_asm_so(i32x4_t r, uint32_t lds, uint32_t voff, uint32_t soff) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds);
  const uint32_t so = __builtin_amdgcn_readfirstlane(soff);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %3 offen lds"
               :: "v"(voff), "s"(r), "s"(m), "s"(so) : "memory", "m0");
}

template <bool NT, bool FP8, bool SWIGLU, typename TC, bool ROPE = false>
__device__ __forceinline__ void gemm_pp_body(const GemmArgs &a) {
  static_assert(!ROPE || (!SWIGLU && sizeof(TC) == 2), "the rotary epilogue writes bf16 projections");
  static_assert(NT || !FP8, "fp8 NN weights use the 4-wave kernel");
  constexpr int BMODE = (NT && FP8) ? B_T8 : NT ? B_T16 : B_NN16;
  constexpr int HB = BMODE == B_T8 ? 8192 : 16384;  // B bytes per half-tile stage
  constexpr int R = BMODE == B_T8 ? 6 : 5;          // ring stages: 144 / 160 KiB
  constexpr bool DMA_G0 = BMODE == B_NN16;  // see the issue plan below
  constexpr int ND = (BMODE == B_T8 ? 3 : 4) * (DMA_G0 ? 2 : 1);  // DMA moves per issuing wave per phase
  constexpr int KP = 32;                            // k per phase

  int tm, tn;
  gemm_tile(a, tm, tn);
  const int64_t m0 = (int64_t)tm * BM;
  const int64_t n0 = (int64_t)tn * (SWIGLU ? BN / 2 : BN);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2, wi = wave & 3;
  const int wm = wi >> 1, wn = wi & 1;
  const int arow0 = 128 * grp + 64 * wm;

  // 4 x 8 tiles of v_mfma_f32_16x16x32_bf16 (which sustains a higher rate
  // than the 32x32x16 form on random operands): A tile i = rows 16 i..,
  // B tile j = B^T rows bw0 + brel[j]..
  f32x4 acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.f;

  const int bsz = FP8 ? 1 : 2;
  const i32x4_t ra = rsrc_words(a.A, a.M * a.lda * 2);
  const int64_t brows = NT ? a.N : a.K;
  const i32x4_t rb0 = rsrc_words(a.B0, brows * a.ldb * bsz);
  const i32x4_t rb1 = rsrc_words(SWIGLU ? a.B1 : a.B0, brows * a.ldb * bsz);

  // DMA_G0: only group 0 issues the DMAs (a whole stage per phase, in its
  // load slot), so the computing wave's MFMA issue never queues behind a
  // vector memory instruction; otherwise all 8 waves issue a share
  constexpr int NWD = DMA_G0 ? 4 : 8;
  // DMA sources: one per-lane base per operand plus a uniform stride per
  // block j (wave wd moves blocks b = NWD j + wd).  Rows past M (A), N (NT
  // B) or K (NN B) land past the buffer's end and read zeros; chunks past K
  // (row-major operands) or past N (NN B columns) are sent out of range.
  const int wd = wave & (NWD - 1);
  const int lc16 = (lane & 3) ^ ((lane >> 4) & 3);  // A / bf16 B^T: logical chunk of this lane
  const int lc8 = (lane & 1) ^ ((lane >> 4) & 1);   // fp8 B^T
  const uint32_t abase = (uint32_t)(((m0 + wd * 16 + (lane >> 2)) * a.lda + lc16 * 8) * 2);
  const uint32_t astr = (uint32_t)(16 * NWD * a.lda * 2);
  uint32_t bbase = 0, bstr = 0, bup = 0, bhalf = 0;
  int bkofs = 0, nn_colok = 0;
  if constexpr (BMODE == B_T16) {
    bbase = (uint32_t)(((n0 + wd * 16 + (lane >> 2)) * a.ldb + lc16 * 8) * 2);
    bstr = (uint32_t)(16 * NWD * a.ldb * 2);
    bup = (uint32_t)(128 * a.ldb * 2);
    bkofs = lc16 * 8;
  } else if constexpr (BMODE == B_T8) {
    bbase = (uint32_t)((n0 + wd * 32 + (lane >> 1)) * a.ldb + lc8 * 16);
    bstr = (uint32_t)(32 * NWD * a.ldb);
    bup = (uint32_t)(128 * a.ldb);
    bkofs = lc8 * 16;
  } else {
    // block b: column half b / 8, k rows (b mod 8) * 4 + l / 16; lane slot
    // l % 16 holds logical chunk (l % 16) ^ nnswz(k)
    const int kq = lane >> 4;
    const int lc = (lane & 15) ^ nnswz(kq);
    bbase = (uint32_t)(((int64_t)(wd % 8 * 4 + kq) * a.ldb + n0 + lc * 8) * 2);
    bstr = (uint32_t)(16 * a.ldb * 2);  // +4 blocks within a half (NWD = 4)
    bhalf = SWIGLU ? 0u : 256u;          // column half 1: +128 columns
    const int64_t c0 = n0 + lc * 8, c1 = n0 + (SWIGLU ? 0 : 128) + lc * 8;
    nn_colok = (c0 < a.N ? 1 : 0) | (c1 < a.N ? 2 : 0);
  }
  // DMA of phase q (k0 = 32 q) into a stage; past K the offsets are out of
  // range and read zeros
  auto issue = [&](uint8_t *As, uint8_t *Bs, int64_t k0) __attribute__((always_inline)) {
    const uint32_t kk0 = (uint32_t)k0;
    const bool ka = k0 + lc16 * 8 < a.K;
    const uint32_t la = lds_addr(As), lb = lds_addr(Bs);
#pragma unroll
    for (int j = 0; j < 16 / NWD; ++j)
      dma16_asm(ra, la + (j * NWD + wd) * 1024, ka ? abase + j * astr + kk0 * 2 : OOB);
    if constexpr (BMODE == B_T8) {
      const bool kb = k0 + bkofs < a.K;
#pragma unroll
      for (int j = 0; j < 8 / NWD; ++j) {
        const bool up = SWIGLU && (j * NWD + wd) >= 4;  // blocks 4..7: the up weight
        dma16_asm(up ? rb1 : rb0, lb + (j * NWD + wd) * 1024, kb ? bbase + j * bstr - (up ? bup : 0) + kk0 : OOB);
      }
    } else if constexpr (BMODE == B_T16) {
      const bool kb = k0 + bkofs < a.K;
#pragma unroll
      for (int j = 0; j < 16 / NWD; ++j) {
        const bool up = SWIGLU && (j * NWD + wd) >= 8;  // blocks 8..15: the up weight
        dma16_asm(up ? rb1 : rb0, lb + (j * NWD + wd) * 1024,
                  kb ? bbase + j * bstr - (up ? bup : 0) + kk0 * 2 : OOB);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16 / NWD; ++j) {
        const int b = j * NWD + wd;  // wave-uniform
        const int h = b >> 3;
        const bool ok = (nn_colok >> h) & 1;
        // k rows (b mod 8) * 4 = wd * 4 (in bbase) + 16 (j mod 2) for NWD = 4,
        // or wd * 4 for NWD = 8 (j = h)
        const uint32_t krow_ofs = NWD == 4 ? (uint32_t)(j & 1) * bstr : 0u;
        dma16_asm((SWIGLU && h) ? rb1 : rb0, lb + b * 1024,
                  ok ? bbase + krow_ofs + h * bhalf + kk0 * (uint32_t)(a.ldb * 2) : OOB);
      }
    }
  };

  // Per-lane LDS byte offsets of the fragments.  16x16x32 operands: lane
  // (g = l / 16, i = l % 16) holds row i of a 16-row tile and k 8 g..8 g+7
  // of the phase (logical chunk g of a 64-byte half-tile row).  The A tile
  // (+16 rows) and B tile (brel) parts are immediates; row bases are
  // multiples of 16, so the row swizzles only depend on i.
  const int l16 = lane & 15, g4 = lane >> 4;
  const int bw0 = SWIGLU ? wn * 64 : wn * 128;  // B^T rows of tile j: bw0 + brel[j]
  constexpr int brel[8] = {0, 16, 32, 48, SWIGLU ? 128 : 64, SWIGLU ? 144 : 80, SWIGLU ? 160 : 96,
                           SWIGLU ? 176 : 112};
  const uint32_t aoff = (arow0 + l16) * 64 + ((g4 ^ hswz(l16)) << 4);
  const uint32_t boff = (bw0 + l16) * 64 + ((g4 ^ hswz(l16)) << 4);
  const uint32_t b8off = (bw0 + l16) * 32 + (((g4 >> 1) ^ hswz8(l16)) << 4) + 8 * (g4 & 1);
  // NN B (ds_read_b64_tr_b16): per B tile j, lane (g, i) reads k rows
  // 8 g + 4 s + i / 4 (s immediate) and columns c + 4 (i % 4) of column half
  // (bw0 + brel[j]) / 128
  uint32_t nnoff[8];
  if (BMODE == B_NN16) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int br = bw0 + brel[j];
      const int half = br >> 7, c = br & 127;
      const int nl = c + 4 * (l16 & 3);
      const int k = 8 * g4 + (l16 >> 2);
      nnoff[j] = half * 8192 + k * 256 + (((nl >> 3) ^ nnswz(k)) << 4) + (nl & 7) * 2;
    }
  }

  // fragments of one phase (one k32 step)
  bf16x8_t af[4], bf[8];
  auto load = [&](const uint8_t *As, const uint8_t *Bs) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) af[i] = *reinterpret_cast<const bf16x8_t *>(As + aoff + i * 1024);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (BMODE == B_T16) {
        bf[j] = *reinterpret_cast<const bf16x8_t *>(Bs + boff + brel[j] * 64);
      } else if (BMODE == B_T8) {
        const uint4 w = e4m3x8_to_bf16x8(*reinterpret_cast<const uint2 *>(Bs + b8off + brel[j] * 32));
        bf[j] = *reinterpret_cast<const bf16x8_t *>(&w);
      } else {
        s16x4 v[2];
#pragma unroll
        for (int sidx = 0; sidx < 2; ++sidx)
          v[sidx] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(Bs + nnoff[j] + 4 * sidx * 256));
        bf[j] = __builtin_shufflevector(__builtin_bit_cast(__attribute__((ext_vector_type(4))) __bf16, v[0]),
                                        __builtin_bit_cast(__attribute__((ext_vector_type(4))) __bf16, v[1]),
                                        0, 1, 2, 3, 4, 5, 6, 7);
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the fragments are in registers
  };
  // C^T tiles (B fragment as the A operand): lane (g, i) of tile (i', j)
  // holds output row 16 i' + i and columns (tile column) + 4 g + 0..3
  auto compute = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf[j], af[i], acc[i][j], 0, 0, 0);
  };
  // slot boundary: the scheduling fences keep the MFMAs (register-only
  // instructions, which the memory clobbers do not pin) inside their slot
  auto slot_end = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    barrier_no_fence();
    __builtin_amdgcn_sched_barrier(0);
  };

  // ring stages [A | B]: one array each, so that the compiler sees that DMA
  // targets and fragment sources of different stages never alias (it tracks
  // a few LDS DMA targets individually; more would make its own waits
  // conservative)
  constexpr int SS = 16384 + HB;
  __shared__ __attribute__((aligned(1024))) uint8_t ST0[SS], ST1[SS], ST2[SS], ST3[SS], ST4[SS], ST5[SS];
  auto sa = [&](auto stag) __attribute__((always_inline)) -> uint8_t * {
    constexpr int S = decltype(stag)::value;
    if constexpr (S == 0) return ST0; else if constexpr (S == 1) return ST1; else if constexpr (S == 2) return ST2;
    else if constexpr (S == 3) return ST3; else if constexpr (S == 4) return ST4; else return ST5;
  };
  auto sb = [&](auto stag) __attribute__((always_inline)) -> uint8_t * { return sa(stag) + 16384; };

  const int nph = (int)((a.K + KP - 1) / KP);
  if (!DMA_G0 || grp == 0) {
    issue(ST0, ST0 + 16384, 0);
    issue(ST1, ST1 + 16384, KP);
    issue(ST2, ST2 + 16384, 2 * KP);
    issue(ST3, ST3 + 16384, 3 * KP);
    issue(ST4, ST4 + 16384, 4 * KP);
    if constexpr (R > 5) issue(ST5, ST5 + 16384, 5 * KP);
  }
  wait_vmem_but<ND * (R - 1)>();  // phase 0 landed
  slot_end();
  if (grp == 0) load(ST0, ST0 + 16384);
  slot_end();
  // phase p in stage S = p mod R; G = this wave's group
  auto phase = [&](auto stag, int p, auto gtag) __attribute__((always_inline)) {
    constexpr int S = decltype(stag)::value;
    constexpr int G = decltype(gtag)::value;
    uint8_t *As = sa(Int<S>{}), *Bs = sb(Int<S>{});
    const uint8_t *An = sa(Int<(S + 1) % R>{}), *Bn = sb(Int<(S + 1) % R>{});
    if (G == 0) compute(); else load(As, Bs);
    wait_vmem_but<ND * (R - 2)>();  // phase p + 1 landed
    slot_end();
    // group 0 reads the next phase unconditionally (past the last phase it
    // reads a stage nothing will consume), then every wave refills stage S
    if (G == 0) load(An, Bn);
    if (!DMA_G0 || G == 0) issue(As, Bs, (int64_t)(p + R) * KP);
    if (G == 1) compute();
    slot_end();
  };
  auto run = [&](auto gtag) __attribute__((always_inline)) {
    int p = 0;
    for (; p + R <= nph; p += R) {
      phase(Int<0>{}, p, gtag);
      phase(Int<1>{}, p + 1, gtag);
      phase(Int<2>{}, p + 2, gtag);
      phase(Int<3>{}, p + 3, gtag);
      phase(Int<4>{}, p + 4, gtag);
      if constexpr (R > 5) phase(Int<5>{}, p + 5, gtag);
    }
    if (p < nph) phase(Int<0>{}, p, gtag);
    if (p + 1 < nph) phase(Int<1>{}, p + 1, gtag);
    if (p + 2 < nph) phase(Int<2>{}, p + 2, gtag);
    if (p + 3 < nph) phase(Int<3>{}, p + 3, gtag);
    if constexpr (R > 5)
      if (p + 4 < nph) phase(Int<4>{}, p + 4, gtag);
  };
  if (grp == 0)
    run(Int<0>{});
  else
    run(Int<1>{});
  wait_vmem();
  if constexpr (ROPE) {
    if (n0 + bw0 < (int64_t)a.rope_nq + a.rope_nk) {
      gemm_epilogue_rope<4>(a, acc, m0 + arow0, n0 + bw0, lane);
      return;
    }
  }
  gemm_epilogue16<SWIGLU, TC, 4>(a, acc, m0 + arow0, n0 + bw0, lane);
}

// ---------------------------------------------------------------------------
// 8-wave kernel with 64-deep K stages (fp8 NT weights)
// ---------------------------------------------------------------------------
// The ping-pong of gemm_pp_body (phases of 32 k, group 0 and group 1
// alternating between MFMAs and fragment reads), but LDS holds a ring of
// three stages of 64 k: A 256 rows x 128 bytes and fp8 B^T 256 rows x 64
// bytes (48 KiB, 144 KiB for the ring).  Each global -> LDS move then reads
// whole 128-byte A lines and 64-byte B row segments: half as many requests
// as 32-deep stages, whose 64- and 32-byte segments kept the texture address
// unit stalled on the L1 cache for a third of the kernel.
//   A stage:  row r, logical 16-byte chunk c (k 8c..8c+7) at slot c ^ ((r >> 1) & 7)
//   B stage:  row r, logical chunk c (k 16c..16c+15) at slot c ^ ((r >> 2) & 3)
// A fragment read (16 rows x one chunk per 16 lanes) and a B read (16 rows
// x one chunk x two halves per 32 lanes) each cover distinct 16- / 8-byte
// groups of a 256-byte LDS row of banks.
// Stage t (phases 2t, 2t + 1) is read by group 0 in the slots before its
// phases and by group 1 in the first slot of each; it is refilled with
// block t + 3 in the second slot of phase 2t + 1.
__device__ __forceinline__ int swz_a64(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int swz_b64(int r) { return (r >> 2) & 3; }

// R16: the kernel stages its bf16 output through LDS (gemm_epilogue_lds;
// launched when the flag GEMM_ROWS16 holds).  A separate kernel, so that
// one epilogue's live values do not add to the other's register pressure.
template <bool SWIGLU, typename TC, bool ROPE = false, bool R16 = false>
__device__ __forceinline__ void gemm_pp64_body(const GemmArgs &a) {
  static_assert(!R16 || sizeof(TC) == 2, "the staged epilogue writes bf16");
  static_assert(!ROPE || (!SWIGLU && sizeof(TC) == 2), "the rotary epilogue writes bf16 projections");
  constexpr int R2 = 3;                         // ring stages
  constexpr int KB = 64;                        // k per stage
  constexpr int SA = 32768, SS = SA + 16384;    // A bytes, stage bytes
  constexpr int NAM = 4, NBM = 2;               // A / B moves per wave per stage
  constexpr int ND = NAM + NBM;

  int tm, tn;
  gemm_tile(a, tm, tn);
  const int64_t m0 = (int64_t)tm * BM;
  const int64_t n0 = (int64_t)tn * (SWIGLU ? BN / 2 : BN);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2, wi = wave & 3;
  const int wm = wi >> 1, wn = wi & 1;
  const int arow0 = 128 * grp + 64 * wm;

  f32x4 acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.f;

  const i32x4_t ra = rsrc_words(a.A, a.M * a.lda * 2);
  const i32x4_t rb0 = rsrc_words(a.B0, a.N * a.ldb);
  const i32x4_t rb1 = rsrc_words(SWIGLU ? a.B1 : a.B0, a.N * a.ldb);

  // A move m = 8 j + wave (j < 4): rows 8 m .. 8 m + 7; lane l fills slot
  // l & 7 of row 8 m + l / 8 with logical chunk (l & 7) ^ swz_a64(row), and
  // swz_a64(row) = (4 m + l / 16) & 7 = (4 wave + l / 16) & 7 for every j.
  const int ac = (lane & 7) ^ ((4 * wave + (lane >> 4)) & 7);
  const uint32_t abase = (uint32_t)(((m0 + 8 * wave + (lane >> 3)) * a.lda + ac * 8) * 2);
  const uint32_t astr = (uint32_t)(64 * a.lda * 2);
  // B move m = 8 j + wave (j < 2): tile rows 16 m .. 16 m + 15; lane l fills
  // slot l & 3 of row 16 m + l / 4 with logical chunk (l & 3) ^ swz_b64(row),
  // swz_b64(row) = (l / 16) & 3.  Tile row r is weight row n0 + r (SwiGLU:
  // rows 128.. are the up weight's rows n0 + r - 128, i.e. move j = 1).
  const int bc = (lane & 3) ^ ((lane >> 4) & 3);
  const uint32_t bbase = (uint32_t)((n0 + 16 * wave + (lane >> 2)) * a.ldb + bc * 16);
  const uint32_t bstr = SWIGLU ? 0u : (uint32_t)(128 * a.ldb);
  // per-lane offset (the base, or OOB for a chunk past K: OOB plus the
  // uniform part stays past the end) plus a uniform per-move part
  auto issue = [&](uint8_t *St, int64_t k0) __attribute__((always_inline)) {
    const uint32_t kk0 = (uint32_t)k0;
    const uint32_t va = k0 + ac * 8 < a.K ? abase : OOB;
    const uint32_t vb = k0 + bc * 16 < a.K ? bbase : OOB;
    const uint32_t la = lds_addr(St), lb = la + SA;
#pragma unroll
    for (int j = 0; j < NAM; ++j) dma16_asm_so(ra, la + (j * 8 + wave) * 1024, va, j * astr + kk0 * 2);
#pragma unroll
    for (int j = 0; j < NBM; ++j)
      dma16_asm_so((SWIGLU && j) ? rb1 : rb0, lb + (j * 8 + wave) * 1024, vb, j * bstr + kk0);
  };

  // fragment offsets of phase half h: A tile i = rows arow0 + 16 i + l16
  // (swz_a64 of those rows = (l16 >> 1) & 7), B tile j = rows bw0 + brel[j]
  // + l16 (swz_b64 = (l16 >> 2) & 3)
  const int l16 = lane & 15, g4 = lane >> 4;
  const int bw0 = SWIGLU ? wn * 64 : wn * 128;
  constexpr int brel[8] = {0, 16, 32, 48, SWIGLU ? 128 : 64, SWIGLU ? 144 : 80, SWIGLU ? 160 : 96,
                           SWIGLU ? 176 : 112};
  // half 1 reads logical chunks 4 + g (A) and 2 + g / 2 (B): slot XOR 4 / 2,
  // i.e. offset bit 6 / bit 5 (the row and lane parts sit in other bits)
  const uint32_t aoff0 = (arow0 + l16) * 128 + ((g4 ^ swz_a64(l16)) << 4);
  const uint32_t boff0 = SA + (bw0 + l16) * 64 + (((g4 >> 1) ^ swz_b64(l16)) << 4) + 8 * (g4 & 1);

  // One LDS base per operand and call, kept opaque so that it is formed at
  // the read (stage bases past 64 KiB do not fit the reads' immediate
  // offsets; hoisted per-stage, per-tile addresses would not fit the
  // register budget); the tile offsets are immediates.
  typedef __attribute__((address_space(3))) const uint8_t lds_u8;
  typedef __attribute__((address_space(3))) const bf16x8_t lds_bf16x8;
  typedef __attribute__((address_space(3))) const unsigned long long lds_u64;
  bf16x8_t af[4], bf[8];
  auto load = [&](const uint8_t *St, auto htag) __attribute__((always_inline)) {
    constexpr int H = decltype(htag)::value;
    // the lane offsets pass through an empty asm first, so that stage base
    // plus offset is formed here and not hoisted out of the loop (six
    // loop-invariant sums would otherwise stay live across it)
    uint32_t ao = H ? (aoff0 ^ 64u) : aoff0, bo = H ? (boff0 ^ 32u) : boff0;
    asm volatile("" : "+v"(ao), "+v"(bo));
    lds_u8 *pa = (lds_u8 *)St + ao;
    lds_u8 *pb = (lds_u8 *)St + bo;
    asm volatile("" : "+v"(pa), "+v"(pb));
#pragma unroll
    for (int i = 0; i < 4; ++i) af[i] = *reinterpret_cast<lds_bf16x8 *>(pa + i * 2048);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const unsigned long long q = *reinterpret_cast<lds_u64 *>(pb + brel[j] * 64);
      const uint4 w = e4m3x8_to_bf16x8(make_uint2((uint32_t)q, (uint32_t)(q >> 32)));
      bf[j] = *reinterpret_cast<const bf16x8_t *>(&w);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  };
  auto compute = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf[j], af[i], acc[i][j], 0, 0, 0);
  };
  auto slot_end = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    barrier_no_fence();
    __builtin_amdgcn_sched_barrier(0);
  };

  // one ring (the DMA is inline asm, which the compiler does not track, and
  // the fragment reads go through opaque bases), reused by the epilogue
  __shared__ __attribute__((aligned(1024))) uint8_t RING[R2 * SS];
  uint8_t *const SG0 = RING, *const SG1 = RING + SS, *const SG2 = RING + 2 * SS;
  auto st = [&](auto stag) __attribute__((always_inline)) -> uint8_t * {
    constexpr int S = decltype(stag)::value;
    if constexpr (S == 0) return SG0; else if constexpr (S == 1) return SG1; else return SG2;
  };

  const int nblk = (int)((a.K + KB - 1) / KB);
  issue(SG0, 0);
  issue(SG1, KB);
  issue(SG2, 2 * KB);
  wait_vmem_but<ND * 2>();  // block 0 landed
  slot_end();
  if (grp == 0) load(SG0, Int<0>{});
  slot_end();
  // phase (block t, half H) in stage S = t mod 3; G = this wave's group
  auto phase = [&](auto stag, auto htag, int t, auto gtag) __attribute__((always_inline)) {
    constexpr int S = decltype(stag)::value;
    constexpr int H = decltype(htag)::value;
    constexpr int G = decltype(gtag)::value;
    uint8_t *Sc = st(Int<S>{});
    if (G == 0) compute(); else load(Sc, Int<H>{});
    if (H == 1) wait_vmem_but<ND * (R2 - 2)>();  // block t + 1 landed
    slot_end();
    // group 0 reads the next phase (past the last block it reads a stage
    // nothing will consume); after the second half every wave refills S
    if (G == 0) {
      if constexpr (H == 0) load(Sc, Int<1>{}); else load(st(Int<(S + 1) % R2>{}), Int<0>{});
    }
    if (H == 1) issue(Sc, (int64_t)(t + R2) * KB);
    if (G == 1) compute();
    slot_end();
  };
  auto run = [&](auto gtag) __attribute__((always_inline)) {
    int t = 0;
    for (; t + R2 <= nblk; t += R2) {
      phase(Int<0>{}, Int<0>{}, t, gtag);
      phase(Int<0>{}, Int<1>{}, t, gtag);
      phase(Int<1>{}, Int<0>{}, t + 1, gtag);
      phase(Int<1>{}, Int<1>{}, t + 1, gtag);
      phase(Int<2>{}, Int<0>{}, t + 2, gtag);
      phase(Int<2>{}, Int<1>{}, t + 2, gtag);
    }
    if (t < nblk) {
      phase(Int<0>{}, Int<0>{}, t, gtag);
      phase(Int<0>{}, Int<1>{}, t, gtag);
    }
    if (t + 1 < nblk) {
      phase(Int<1>{}, Int<0>{}, t + 1, gtag);
      phase(Int<1>{}, Int<1>{}, t + 1, gtag);
    }
  };
  if (grp == 0)
    run(Int<0>{});
  else
    run(Int<1>{});
  wait_vmem();
  if constexpr (ROPE && R16) {
    barrier_no_fence();  // the ring is idle
    gemm_epilogue_rope_lds<4>(a, acc, m0, n0, arow0, bw0, lane, RING);
    return;
  } else if constexpr (ROPE) {
    if (n0 + bw0 < (int64_t)a.rope_nq + a.rope_nk) {
      gemm_epilogue_rope<4>(a, acc, m0 + arow0, n0 + bw0, lane);
      return;
    }
  } else if constexpr (R16) {
    barrier_no_fence();  // every wave's DMA has landed and its fragment reads are done: the ring is idle
    gemm_epilogue_lds<SWIGLU, 4>(a, acc, m0, n0, arow0, bw0, lane, RING);
    return;
  }
  gemm_epilogue16<SWIGLU, TC, 4>(a, acc, m0 + arow0, n0 + bw0, lane);
}

// ---------------------------------------------------------------------------
// 8-wave kernel with 64-deep A stages (bf16 K x N weights)
// ---------------------------------------------------------------------------
// The ping-pong of gemm_pp_body for NN bf16 weights, with A in the 64-deep
// ring of gemm_pp64_body (three 64-k blocks, 256 rows x 128 bytes, 96 KiB)
// and B in a ring of four 32-k phases in the NN layout of gemm_pp_body
// (32 k rows x 256 columns, 64 KiB; 160 KiB in all).  A moves read whole
// 128-byte lines of 8 rows instead of 64-byte halves of 16 rows; B moves
// read 256-byte runs of k rows as before.  Phase q (block t = q / 2, half
// H = q mod 2) reads A stage t mod 3 and B stage q mod 4, the fragments and
// MFMA order of the 32-deep kernel (bit-identical results).  After phase q
// each wave refills B stage q mod 4 with phase q + 4 and, after the second
// half, A stage t mod 3 with block t + 3.
template <bool SWIGLU, typename TC, bool R16 = false>
__device__ __forceinline__ void gemm_nn64_body(const GemmArgs &a) {
  static_assert(!R16 || sizeof(TC) == 2, "the staged epilogue writes bf16");
  constexpr int RA = 3;                       // A ring stages (one block each)
  constexpr int KB = 64, KP = 32;             // k per block, per phase
  constexpr int SA = 32768, SP = 16384;       // A stage bytes, B stage bytes (one phase)
  constexpr int BOFF = RA * SA;               // the B ring follows the A ring
  constexpr int NAM = 4, NBM = 2;             // moves per wave: A per block, B per phase

  int tm, tn;
  gemm_tile(a, tm, tn);
  const int64_t m0 = (int64_t)tm * BM;
  const int64_t n0 = (int64_t)tn * (SWIGLU ? BN / 2 : BN);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2, wi = wave & 3;
  const int wm = wi >> 1, wn = wi & 1;
  const int arow0 = 128 * grp + 64 * wm;

  f32x4 acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.f;

  const i32x4_t ra = rsrc_words(a.A, a.M * a.lda * 2);
  const i32x4_t rb0 = rsrc_words(a.B0, a.K * a.ldb * 2);
  const i32x4_t rb1 = rsrc_words(SWIGLU ? a.B1 : a.B0, a.K * a.ldb * 2);

  // A move m = 8 j + wave (j < 4): rows 8 m .. 8 m + 7, lane l fills slot
  // l & 7 of row 8 m + l / 8 with logical chunk (l & 7) ^ swz_a64(row) =
  // (l & 7) ^ ((4 wave + l / 16) & 7).
  const int ac = (lane & 7) ^ ((4 * wave + (lane >> 4)) & 7);
  const uint32_t abase = (uint32_t)(((m0 + 8 * wave + (lane >> 3)) * a.lda + ac * 8) * 2);
  const uint32_t astr = (uint32_t)(64 * a.lda * 2);
  // B move j (j < 2) of wave w: column half j, k rows 4 w + l / 16 of the
  // phase; lane slot l % 16 holds logical chunk (l % 16) ^ nnswz(k) (8
  // columns each).  k rows past K lie past the buffer's end and read zeros;
  // chunks past N are sent out of range.  SwiGLU: half 1 is the up weight's
  // columns n0 ...
  const int kq = lane >> 4;
  const int lc = (lane & 15) ^ nnswz(kq);
  const uint32_t bbase = (uint32_t)(((int64_t)(4 * wave + kq) * a.ldb + n0 + lc * 8) * 2);
  const uint32_t bb0 = n0 + lc * 8 < a.N ? bbase : OOB;
  const uint32_t bb1 = n0 + (SWIGLU ? 0 : 128) + lc * 8 < a.N ? bbase + (SWIGLU ? 0u : 256u) : OOB;
  auto issue_a = [&](const uint8_t *St, int64_t k0) __attribute__((always_inline)) {
    const uint32_t va = k0 + ac * 8 < a.K ? abase : OOB;
    const uint32_t la = lds_addr(St);
#pragma unroll
    for (int j = 0; j < NAM; ++j) dma16_asm_so(ra, la + (j * 8 + wave) * 1024, va, j * astr + (uint32_t)k0 * 2);
  };
  auto issue_b = [&](const uint8_t *St, int64_t k0) __attribute__((always_inline)) {
    const uint32_t lb = lds_addr(St);
    const uint32_t kofs = (uint32_t)k0 * (uint32_t)(a.ldb * 2);
    dma16_asm_so(rb0, lb + wave * 1024, bb0, kofs);
    dma16_asm_so(SWIGLU ? rb1 : rb0, lb + (8 + wave) * 1024, bb1, kofs);
  };

  // Per-lane fragment offsets.  A (64-deep stage, phase half H): tile i =
  // rows arow0 + 16 i + l16, chunk g ^ swz_a64 (half 1: slot XOR 4, offset
  // bit 6).  B (ds_read_b64_tr_b16): per B tile j, lane (g, i) reads k rows
  // 8 g + 4 s + i / 4 (s immediate) and columns c + 4 (i % 4) of column half
  // (bw0 + brel[j]) / 128.
  const int l16 = lane & 15, g4 = lane >> 4;
  const int bw0 = SWIGLU ? wn * 64 : wn * 128;
  constexpr int brel[8] = {0, 16, 32, 48, SWIGLU ? 128 : 64, SWIGLU ? 144 : 80, SWIGLU ? 160 : 96,
                           SWIGLU ? 176 : 112};
  const uint32_t aoff0 = (arow0 + l16) * 128 + ((g4 ^ swz_a64(l16)) << 4);
  uint32_t nnoff[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int br = bw0 + brel[j];
    const int half = br >> 7, c = br & 127;
    const int nl = c + 4 * (l16 & 3);
    const int k = 8 * g4 + (l16 >> 2);
    nnoff[j] = half * 8192 + k * 256 + (((nl >> 3) ^ nnswz(k)) << 4) + (nl & 7) * 2;
  }

  typedef __attribute__((address_space(3))) const uint8_t lds_u8;
  typedef __attribute__((address_space(3))) const bf16x8_t lds_bf16x8;
  bf16x8_t af[4], bf[8];
  auto load = [&](const uint8_t *Sa, const uint8_t *Sb, auto htag) __attribute__((always_inline)) {
    constexpr int H = decltype(htag)::value;
    uint32_t ao = H ? (aoff0 ^ 64u) : aoff0;
    asm volatile("" : "+v"(ao));
    lds_u8 *pa = (lds_u8 *)Sa + ao;
    asm volatile("" : "+v"(pa));
#pragma unroll
    for (int i = 0; i < 4; ++i) af[i] = *reinterpret_cast<lds_bf16x8 *>(pa + i * 2048);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      s16x4 v[2];
#pragma unroll
      for (int sidx = 0; sidx < 2; ++sidx)
        v[sidx] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)((lds_u8 *)Sb + nnoff[j] + 4 * sidx * 256));
      bf[j] = __builtin_shufflevector(__builtin_bit_cast(__attribute__((ext_vector_type(4))) __bf16, v[0]),
                                      __builtin_bit_cast(__attribute__((ext_vector_type(4))) __bf16, v[1]),
                                      0, 1, 2, 3, 4, 5, 6, 7);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  };
  auto compute = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf[j], af[i], acc[i][j], 0, 0, 0);
  };
  auto slot_end = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    barrier_no_fence();
    __builtin_amdgcn_sched_barrier(0);
  };

  // one array for both rings, reused by the epilogue
  __shared__ __attribute__((aligned(1024))) uint8_t RING[RA * SA + 4 * SP];
  uint8_t *const RB = RING + BOFF;

  // Per wave, in issue order: A0, B0, A1, B1, B2, A2, B3, then after phase
  // q the moves X_q = B(q + 4), preceded after a second half (q = 2t + 1) by
  // A(t + 3).  vmcnt counts in issue order, so "phase q + 1 landed" (waited
  // for in phase q, before X_q) leaves X_{q-2} and X_{q-1} outstanding:
  // NAM + 2 NBM moves.
  const int nblk = (int)((a.K + KB - 1) / KB);
  issue_a(RING, 0);
  issue_b(RB, 0);
  issue_a(RING + SA, KB);
  issue_b(RB + SP, KP);
  issue_b(RB + 2 * SP, 2 * KP);
  issue_a(RING + 2 * SA, 2 * KB);
  issue_b(RB + 3 * SP, 3 * KP);
  wait_vmem_but<2 * NAM + 3 * NBM>();  // A0, B0 landed
  slot_end();
  if (grp == 0) load(RING, RB, Int<0>{});
  slot_end();
  // phase (block t, half H) in A stage sa = t mod 3 and B stage sq = (2 t +
  // H) mod 4; G = this wave's group
  auto phase = [&](int sa, int sq, auto htag, int t, auto gtag) __attribute__((always_inline)) {
    constexpr int H = decltype(htag)::value;
    constexpr int G = decltype(gtag)::value;
    const uint8_t *Sa = RING + sa * SA, *Sb = RB + sq * SP;
    if (G == 0) compute(); else load(Sa, Sb, Int<H>{});
    wait_vmem_but<NAM + 2 * NBM>();  // phase 2 t + H + 1 landed
    slot_end();
    // group 0 reads the next phase (past the last block it reads a stage
    // nothing will consume); then every wave refills
    if (G == 0) {
      const uint8_t *Sb1 = RB + ((sq + 1) & 3) * SP;
      if constexpr (H == 0) load(Sa, Sb1, Int<1>{}); else load(RING + (sa == RA - 1 ? 0 : sa + 1) * SA, Sb1, Int<0>{});
    }
    if (H == 1) issue_a(Sa, (int64_t)(t + RA) * KB);
    issue_b(Sb, (int64_t)(2 * t + H + 4) * KP);
    if (G == 1) compute();
    slot_end();
  };
  auto run = [&](auto gtag) __attribute__((always_inline)) {
    int sa = 0, sq = 0;
    for (int t = 0; t < nblk; ++t) {
      phase(sa, sq, Int<0>{}, t, gtag);
      phase(sa, sq + 1, Int<1>{}, t, gtag);
      sa = sa == RA - 1 ? 0 : sa + 1;
      sq ^= 2;
    }
  };
  if (grp == 0)
    run(Int<0>{});
  else
    run(Int<1>{});
  wait_vmem();
  if constexpr (R16) {
    barrier_no_fence();  // every wave's DMA has landed and its fragment reads are done: the ring is idle
    gemm_epilogue_lds<SWIGLU, 4>(a, acc, m0, n0, arow0, bw0, lane, RING);
    return;
  }
  gemm_epilogue16<SWIGLU, TC, 4>(a, acc, m0 + arow0, n0 + bw0, lane);
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

#define NK_GEMM_PP(NT, FP8, SW, TC, name)                                                \
  extern "C" __global__ __launch_bounds__(512, 1) void name(GemmArgs a) {                \
    gemm_pp_body<NT, FP8, SW, TC>(a);                                                    \
  }

NK_GEMM_PP(false, false, false, bf16, nk_gemm8_nn_bf16_bf16)
NK_GEMM_PP(false, false, false, float, nk_gemm8_nn_bf16_f32)
NK_GEMM_PP(true, false, false, bf16, nk_gemm8_nt_bf16_bf16)
NK_GEMM_PP(true, false, false, float, nk_gemm8_nt_bf16_f32)
NK_GEMM_PP(false, false, true, bf16, nk_gemm8_swiglu_nn_bf16_bf16)
NK_GEMM_PP(true, false, true, bf16, nk_gemm8_swiglu_nt_bf16_bf16)
NK_GEMM_PP(true, true, false, bf16, nk_gemm8_nt_e4m3_bf16)
NK_GEMM_PP(true, true, false, float, nk_gemm8_nt_e4m3_f32)
NK_GEMM_PP(true, true, true, bf16, nk_gemm8_swiglu_nt_e4m3_bf16)

// fused QKV projection with the rotary embedding of q and k
#define NK_GEMM_ROPE(NT, FP8, name)                                                      \
  extern "C" __global__ __launch_bounds__(512, 1) void name(GemmArgs a) {                \
    gemm_pp_body<NT, FP8, false, bf16, true>(a);                                         \
  }

#define NK_GEMM_K64(SW, TC, ROPE, R16, name)                                             \
  extern "C" __global__ __launch_bounds__(512, 1) void name(GemmArgs a) {                \
    gemm_pp64_body<SW, TC, ROPE, R16>(a);                                                \
  }

NK_GEMM_K64(false, bf16, false, false, nk_gemm8k_nt_e4m3_bf16)
NK_GEMM_K64(false, float, false, false, nk_gemm8k_nt_e4m3_f32)
NK_GEMM_K64(true, bf16, false, false, nk_gemm8k_swiglu_nt_e4m3_bf16)
NK_GEMM_K64(false, bf16, true, false, nk_gemm8k_nt_e4m3_bf16_rope)
NK_GEMM_K64(false, bf16, false, true, nk_gemm8k_nt_e4m3_bf16_r16)
NK_GEMM_K64(true, bf16, false, true, nk_gemm8k_swiglu_nt_e4m3_bf16_r16)
NK_GEMM_K64(false, bf16, true, true, nk_gemm8k_nt_e4m3_bf16_rope_r16)

#define NK_GEMM_NN64(SW, TC, R16, name)                                                  \
  extern "C" __global__ __launch_bounds__(512, 1) void name(GemmArgs a) {                \
    gemm_nn64_body<SW, TC, R16>(a);                                                      \
  }

NK_GEMM_NN64(false, bf16, false, nk_gemm8k_nn_bf16_bf16)
NK_GEMM_NN64(false, float, false, nk_gemm8k_nn_bf16_f32)
NK_GEMM_NN64(true, bf16, false, nk_gemm8k_swiglu_nn_bf16_bf16)
NK_GEMM_NN64(false, bf16, true, nk_gemm8k_nn_bf16_bf16_r16)
NK_GEMM_NN64(true, bf16, true, nk_gemm8k_swiglu_nn_bf16_bf16_r16)

// Split-K entries for short M (a decode batch, a short prefill), where the
// 256 x 256 tiles leave most CUs idle: workgroup (tile, s) computes the
// tile's fp32 partial sum over K range s with the unchanged body, handed the
// range as its operands: A and B advanced to the range's first k, K = the
// range's length, C = the range's partial plane (flags: at most GEMM_VEC,
// so the epilogue stores the plain sums).  The bodies' buffer ranges
// then end where the range ends (rows of NN B, columns of A and NT B past
// it read zeros, as at a real K end), and the ranges' planes are added in
// order by the reduction kernel of gemv.hip, which applies the epilogue.
template <bool NT, int BSZ>
__device__ __forceinline__ GemmArgs splitk_args(const GemmArgs &a) {
  GemmArgs s = a;
  const int64_t k0 = (int64_t)blockIdx.y * a.kc;
  s.K = min((int64_t)a.kc, a.K - k0);
  s.A = reinterpret_cast<const uint16_t *>(a.A) + k0;
  s.B0 = reinterpret_cast<const uint8_t *>(a.B0) + (NT ? k0 * BSZ : k0 * a.ldb * BSZ);
  s.C = reinterpret_cast<float *>(a.C) + (int64_t)blockIdx.y * a.M * a.ldc;
  return s;
}

extern "C" __global__ __launch_bounds__(512, 1) void nk_gemm8k_nn_bf16_f32_splitk(GemmArgs a) {
  gemm_nn64_body<false, float, false>(splitk_args<false, 2>(a));
}
extern "C" __global__ __launch_bounds__(512, 1) void nk_gemm8_nt_bf16_f32_splitk(GemmArgs a) {
  gemm_pp_body<true, false, false, float>(splitk_args<true, 2>(a));
}
extern "C" __global__ __launch_bounds__(512, 1) void nk_gemm8k_nt_e4m3_f32_splitk(GemmArgs a) {
  gemm_pp64_body<false, float, false, false>(splitk_args<true, 1>(a));
}

NK_GEMM_ROPE(false, false, nk_gemm8_nn_bf16_bf16_rope)
NK_GEMM_ROPE(true, false, nk_gemm8_nt_bf16_bf16_rope)
NK_GEMM_ROPE(true, true, nk_gemm8_nt_e4m3_bf16_rope)
