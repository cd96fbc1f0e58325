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

#define BM 256
#define BN 256
#define BK 64
#define NTHREADS 256
#define GROUP_M 8

enum {
  GEMM_BIAS = 1,      // + bias[col] (bf16)
  GEMM_SCALE = 2,     // * scale[col] (fp32), per output column (fp8 weights)
  GEMM_RESID = 4,     // + residual[row][col] (same dtype as C)
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
};
template <> struct OutT<float> {
  static __device__ __forceinline__ void store(void *C, int64_t i, float v) {
    reinterpret_cast<float *>(C)[i] = v;
  }
  static __device__ __forceinline__ float load(const void *C, int64_t i) {
    return reinterpret_cast<const float *>(C)[i];
  }
};

// half-word i (0..7) of an 8 x bf16 vector
__device__ __forceinline__ uint32_t h16(const uint4 &v, int i) {
  uint32_t w = (i < 2) ? v.x : (i < 4) ? v.y : (i < 6) ? v.z : v.w;
  return (i & 1) ? (w >> 16) : (w & 0xffffu);
}

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// ---------------------------------------------------------------------------
// global -> register staging
// ---------------------------------------------------------------------------
// A tile: 256 rows x 64 k = 2048 chunks of 8 bf16; 8 per thread.
struct StageA {
  uint4 r[8];
};

__device__ __forceinline__ void load_a(StageA &s, const GemmArgs &a, int64_t m0, int64_t k0) {
  const uint16_t *A = reinterpret_cast<const uint16_t *>(a.A);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = threadIdx.x + NTHREADS * i;
    const int row = c >> 3, kc = c & 7;
    const int64_t m = m0 + row, k = k0 + kc * 8;
    if (m < a.M && k < a.K)
      s.r[i] = *reinterpret_cast<const uint4 *>(A + m * a.lda + k);
    else
      s.r[i] = make_uint4(0, 0, 0, 0);
  }
}

__device__ __forceinline__ void store_a(const StageA &s, uint16_t *As) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = threadIdx.x + NTHREADS * i;
    const int row = c >> 3, kc = c & 7;
    *reinterpret_cast<uint4 *>(As + row * BK + swz(row, kc) * 8) = s.r[i];
  }
}

// B tile staged as B^T[256 n][64 k].
template <bool NT, bool FP8>
struct StageB {
  // NT: 8 chunks of 8 k (one n row each); NN: 8 k rows x 8 n of one n chunk
  uint4 r[8];
};

// column (n) of the B^T tile row `nt` (0..255) -> (matrix, global column)
template <bool SWIGLU>
__device__ __forceinline__ const void *b_src(const GemmArgs &a, int nt, int64_t n0, int64_t &col) {
  if (SWIGLU) {
    col = n0 + (nt & 127);
    return nt < 128 ? a.B0 : a.B1;
  }
  col = n0 + nt;
  return a.B0;
}

template <bool NT, bool FP8, bool SWIGLU>
__device__ __forceinline__ void load_b(StageB<NT, FP8> &s, const GemmArgs &a, int64_t n0, int64_t k0) {
  if (NT) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = threadIdx.x + NTHREADS * i;
      const int nt = c >> 3, kc = c & 7;
      int64_t col;
      const void *B = b_src<SWIGLU>(a, nt, n0, col);
      const int64_t k = k0 + kc * 8;
      if (col < a.N && k < a.K) {
        if (FP8) {
          uint2 q = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint8_t *>(B) + col * a.ldb + k);
          s.r[i] = e4m3x8_to_bf16x8(q);
        } else {
          s.r[i] = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(B) + col * a.ldb + k);
        }
      } else {
        s.r[i] = make_uint4(0, 0, 0, 0);
      }
    }
  } else {
    // thread -> (k block of 8 rows, n chunk of 8 columns)
    const int kb = threadIdx.x >> 5, nc = threadIdx.x & 31;
    int64_t col;
    const void *B = b_src<SWIGLU>(a, nc * 8, n0, col);
    uint4 in[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t k = k0 + kb * 8 + j;
      if (k < a.K && col < a.N) {
        if (FP8) {
          uint2 q = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint8_t *>(B) + k * a.ldb + col);
          in[j] = e4m3x8_to_bf16x8(q);
        } else {
          in[j] = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(B) + k * a.ldb + col);
        }
      } else {
        in[j] = make_uint4(0, 0, 0, 0);
      }
    }
    // 8 x 8 transpose: r[i] = the 8 k values of column nc*8 + i
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t w[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) w[p] = h16(in[2 * p], i) | (h16(in[2 * p + 1], i) << 16);
      s.r[i] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

template <bool NT, bool FP8>
__device__ __forceinline__ void store_b(const StageB<NT, FP8> &s, uint16_t *Bs) {
  if (NT) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = threadIdx.x + NTHREADS * i;
      const int nt = c >> 3, kc = c & 7;
      *reinterpret_cast<uint4 *>(Bs + nt * BK + swz(nt, kc) * 8) = s.r[i];
    }
  } else {
    const int kb = threadIdx.x >> 5, nc = threadIdx.x & 31;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int nt = nc * 8 + i;
      *reinterpret_cast<uint4 *>(Bs + nt * BK + swz(nt, kb) * 8) = s.r[i];
    }
  }
}

// ---------------------------------------------------------------------------
// main kernel
// ---------------------------------------------------------------------------
template <bool NT, bool FP8, bool SWIGLU, typename TC>
__device__ __forceinline__ void gemm_body(const GemmArgs &a) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * BK];

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
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, lhi = lane >> 5;

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

  StageA sa;
  StageB<NT, FP8> sb;
  const int ktiles = (int)((a.K + BK - 1) / BK);
  load_a(sa, a, m0, 0);
  load_b<NT, FP8, SWIGLU>(sb, a, n0, 0);
  store_a(sa, As[0]);
  store_b<NT, FP8>(sb, Bs[0]);
  __syncthreads();

  for (int t = 0; t < ktiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ktiles) {
      load_a(sa, a, m0, (int64_t)(t + 1) * BK);
      load_b<NT, FP8, SWIGLU>(sb, a, n0, (int64_t)(t + 1) * BK);
    }
    const uint16_t *as = As[buf];
    const uint16_t *bs = Bs[buf];
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int chunk = kk * 2 + lhi;
      bf16x8_t af[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = wm * 128 + i * 32 + l32;
        af[i] = *reinterpret_cast<const bf16x8_t *>(as + row * BK + swz(row, chunk) * 8);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = brow[j] + l32;
        bfr[j] = *reinterpret_cast<const bf16x8_t *>(bs + row * BK + swz(row, chunk) * 8);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (t + 1 < ktiles) {
      store_a(sa, As[buf ^ 1]);
      store_b<NT, FP8>(sb, Bs[buf ^ 1]);
    }
    __syncthreads();
  }

  // epilogue: lane holds column l32 of each 32 x 32 tile and rows
  // (r / 4) * 8 + lhi * 4 + r % 4
  if (SWIGLU) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t col = n0 + wn * 64 + j * 32 + l32;
        if (col >= a.N) continue;
        const float sg = (a.flags & GEMM_SCALE) ? a.scale0[col] : 1.f;
        const float su = (a.flags & GEMM_SCALE) ? a.scale1[col] : 1.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm * 128 + i * 32 + (r >> 2) * 8 + lhi * 4 + (r & 3);
          if (row < a.M) {
            const float g = acc[i][j][r] * sg;
            const float u = acc[i][j + 2][r] * su;
            const float h = g * (1.0f / (1.0f + expf(-g))) * u;
            OutT<TC>::store(a.C, row * a.ldc + col, h);
          }
        }
      }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t col = n0 + wn * 128 + j * 32 + l32;
        if (col >= a.N) continue;
        const float sc = (a.flags & GEMM_SCALE) ? a.scale0[col] : 1.f;
        const float bi = (a.flags & GEMM_BIAS) ? bf16_to_f32(reinterpret_cast<const uint16_t *>(a.bias)[col]) : 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm * 128 + i * 32 + (r >> 2) * 8 + lhi * 4 + (r & 3);
          if (row < a.M) {
            float v = acc[i][j][r] * sc + bi;
            if (a.flags & GEMM_RESID) v += OutT<TC>::load(a.resid, row * a.ldc + col);
            OutT<TC>::store(a.C, row * a.ldc + col, v);
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
