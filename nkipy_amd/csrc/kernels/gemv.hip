// Projections of a few rows (M <= 8 on the VALU, M <= 32 on MFMA; a decode
// token per sequence) on gfx950: C[M, N] = A[M, K] @ B with the epilogues of
// the MFMA GEMM (gemm.hip).
//
// At such M the GEMM's 256-row tiles compute mostly padding and its grid
// has N / 256 workgroups: a token's projection is weight streaming, bound by
// HBM.  Here the K dimension is cut into ksplit ranges so that the grid
// fills the part, and each workgroup streams its slice of the weights once:
//   nk_gemv_{nn,nt}_{bf16,e4m3}[_swiglu]   partial sums over one K range
//       into an fp32 workspace P[split][m][n] (a second array for the up
//       weights of the SwiGLU form);
//   nk_gemv_mfma_{nn_bf16,nt_bf16,nt_e4m3}[_swiglu]_t{1,2}   the same on
//       16-row MFMA tiles (below);
//   nk_gemv_out_{bf16,f32}[_swiglu]        the splits added in a fixed order,
//       then the epilogue (per-column scale, bias, bf16 roundings, residual;
//       or silu(g) u) as the GEMM's, and the store.
// fp32 accumulation throughout; fp8 codes are decoded exactly (e4m3 fits in
// fp32) and scaled in the epilogue, as in the GEMM.
//
// Products are v_dot2_f32_bf16 (two bf16 products of a packed pair added
// to an fp32 accumulator: two multiply-adds per lane-instruction, operands
// used as stored).
// NN (B is K x N, row-major, ldb): a workgroup owns 256 columns and one K
// range.  Thread t: column chunk t / 8 (8 columns), k lane t % 8 (rows
// k0 + t % 8 + 16 j and the row 8 below it, a pair for the dot products);
// a wave's load of one row step covers 8 rows x 128 bytes (bf16) or 64
// bytes (fp8).  A's rows of the range sit in LDS already paired the same
// way (x[k], x[k + 8]).  The 8 k lanes of a chunk are added by a fixed
// shuffle tree.
// NT (B is N x K, row-major, ldb): a workgroup owns 4 waves x NT_ROWS rows
// and one K range; the 64 lanes of a wave take 16-byte chunks of each row
// in turn (1 KiB contiguous per load; consecutive k pair up in each 32-bit
// word, as in A's rows in LDS), the lanes are added by a fixed shuffle
// tree.
// A's rows of the K range sit in LDS as bf16 (M x KC <= 8 x 1024).
// Kernels come for row counts up to MT = 1, 4 and 8 (accumulators sized to
// MT; _m<MT> in the symbol).

#include "common.h"

using namespace nk;

#define GV_MAX_M 8
#define GV_MAX_KC 1024
#define NT_ROWS 4

enum {
  GEMM_BIAS = 1, GEMM_SCALE = 2, GEMM_RESID = 4, GEMM_RND_BIAS = 16, GEMM_RND_RESID = 32,
};

struct GemvArgs {
  const uint16_t *A;     // M x K bf16, row stride lda
  const void *B0;        // weights (NN: K x N; NT: N x K), row stride ldb
  const void *B1;        // up weights (SwiGLU), same layout
  void *C;               // M x N, row stride ldc
  const uint16_t *bias;  // N bf16
  const float *scale0;   // N fp32 (fp8 weights)
  const float *scale1;   // N fp32 (fp8 up weights)
  const void *resid;     // M x N, C dtype, row stride ldc
  float *ws;             // P0 [ksplit][M][N], then P1 (SwiGLU)
  int64_t M, N, K, lda, ldb, ldc;
  int32_t ksplit, kc;    // K ranges of kc (a multiple of 8, or of 16 for NT fp8)
  int32_t flags, pad;
};

// 8 weights of one 16-byte (bf16) or 8-byte (fp8) load as fp32
template <bool FP8> struct W8;
template <> struct W8<false> {
  typedef uint4 raw;
  static __device__ __forceinline__ raw load(const void *p, int64_t e) {
    return *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(p) + e);
  }
  static __device__ __forceinline__ void decode(const raw &w, float (&f)[8]) {
    f[0] = __uint_as_float(w.x << 16); f[1] = __uint_as_float(w.x & 0xffff0000u);
    f[2] = __uint_as_float(w.y << 16); f[3] = __uint_as_float(w.y & 0xffff0000u);
    f[4] = __uint_as_float(w.z << 16); f[5] = __uint_as_float(w.z & 0xffff0000u);
    f[6] = __uint_as_float(w.w << 16); f[7] = __uint_as_float(w.w & 0xffff0000u);
  }
};
template <> struct W8<true> {
  typedef uint2 raw;
  static __device__ __forceinline__ raw load(const void *p, int64_t e) {
    return *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint8_t *>(p) + e);
  }
  static __device__ __forceinline__ void decode(const raw &w, float (&f)[8]) {
    const uint4 b = e4m3x8_to_bf16x8(w);  // exact
    W8<false>::decode(b, f);
  }
};

typedef __bf16 gv_bf16x2 __attribute__((ext_vector_type(2)));
// acc + lo(x) lo(w) + hi(x) hi(w) on packed bf16 pairs
__device__ __forceinline__ float dot2(uint32_t x, uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(gv_bf16x2, x), __builtin_bit_cast(gv_bf16x2, w), acc,
                                         false);
}
// 8 bf16 columns of two k rows -> 8 (row lo, row hi) pairs, column order
__device__ __forceinline__ void pair8(const uint4 &lo, const uint4 &hi, uint32_t (&p)[8]) {
  const uint32_t l[4] = {lo.x, lo.y, lo.z, lo.w}, h[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p[2 * i] = __builtin_amdgcn_perm(h[i], l[i], 0x05040100u);
    p[2 * i + 1] = __builtin_amdgcn_perm(h[i], l[i], 0x07060302u);
  }
}
// raw 8 weights -> 8 bf16 (fp8 decoded exactly)
template <bool FP8>
__device__ __forceinline__ uint4 w8_bf16(const typename W8<FP8>::raw &w) {
  if constexpr (FP8) {
    return e4m3x8_to_bf16x8(w);
  } else {
    return w;
  }
}

// A's rows m < MT of the K range as the NN kernel's pairs: word q of row m
// holds (x[k], x[k + 8]), k = k0 + 16 (q / 8) + q % 8; zero past the range
// (the next range's rows), past K and for rows past M
template <int MT>
__device__ __forceinline__ void stage_a_pairs(const GemvArgs &a, uint32_t *xp, int64_t k0, int np) {
  const int kend = (int)min((int64_t)a.kc, a.K - k0);
  for (int i = threadIdx.x; i < MT * np; i += 256) {
    const int m = i / np, q = i % np;
    const int kl = 16 * (q >> 3) + (q & 7), kh = kl + 8;
    uint32_t lo = 0, hi = 0;
    if (m < a.M) {
      if (kl < kend) lo = a.A[m * a.lda + k0 + kl];
      if (kh < kend) hi = a.A[m * a.lda + k0 + kh];
    }
    xp[m * np + q] = lo | (hi << 16);
  }
}

// A's rows m < MT, columns [k0, k0 + kc) into LDS as bf16: zeros past K and
// for the rows past M, which the kernels then compute with (every
// accumulator loop has a fixed trip count, so the accumulators stay in
// registers) and do not store
template <int MT>
__device__ __forceinline__ void stage_a(const GemvArgs &a, uint16_t *xs, int64_t k0) {
  const int per = a.kc / 8;  // 16-byte chunks per row
  for (int i = threadIdx.x; i < MT * per; i += 256) {
    const int m = i / per, c = i % per;
    const int64_t k = k0 + 8 * c;
    uint4 w = make_uint4(0, 0, 0, 0);
    if (m < a.M && k < a.K) w = *reinterpret_cast<const uint4 *>(a.A + m * a.lda + k);
    *reinterpret_cast<uint4 *>(xs + m * a.kc + 8 * c) = w;
  }
}

template <bool FP8, bool SWIGLU, int MT>
__device__ __forceinline__ void gemv_nn_body(const GemvArgs &a) {
  __shared__ __attribute__((aligned(16))) uint32_t xp[GV_MAX_M * (GV_MAX_KC / 2)];
  const int tid = threadIdx.x;
  const int ks = blockIdx.x % a.ksplit;
  const int64_t n0 = (int64_t)(blockIdx.x / a.ksplit) * 256;
  const int64_t k0 = (int64_t)ks * a.kc;
  const int np = ((a.kc + 15) >> 4) * 8;  // pairs per row of the range
  stage_a_pairs<MT>(a, xp, k0, np);
  __syncthreads();

  const int cc = tid >> 3, kl = tid & 7;
  const int64_t col = n0 + 8 * cc;
  const bool incol = col < a.N;  // N is a multiple of 8
  const int64_t colc = incol ? col : 0;
  const int M = (int)a.M;
  float acc[SWIGLU ? 2 : 1][MT][8];
#pragma unroll
  for (int w = 0; w < (SWIGLU ? 2 : 1); ++w)
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[w][m][e] = 0.f;
  const int kend = (int)min((int64_t)a.kc, a.K - k0);
  // pair j of this lane: rows kl + 16 j and kl + 16 j + 8 of the range (the
  // second zero past the range end)
  for (int kk = kl; kk < kend; kk += 16) {
    const bool two = kk + 8 < kend;
    const int64_t r0 = k0 + kk, r1 = two ? r0 + 8 : r0;
    typename W8<FP8>::raw b0[2], b1[2];
    b0[0] = W8<FP8>::load(a.B0, r0 * a.ldb + colc);
    b0[1] = W8<FP8>::load(a.B0, r1 * a.ldb + colc);
    if constexpr (SWIGLU) {
      b1[0] = W8<FP8>::load(a.B1, r0 * a.ldb + colc);
      b1[1] = W8<FP8>::load(a.B1, r1 * a.ldb + colc);
    }
    const int q = (kk >> 4) * 8 + kl;
    uint32_t wp[8], up[8];
    {
      const uint4 z = make_uint4(0, 0, 0, 0);
      const uint4 hi = w8_bf16<FP8>(b0[1]);
      pair8(w8_bf16<FP8>(b0[0]), two ? hi : z, wp);
      if constexpr (SWIGLU) {
        const uint4 hu = w8_bf16<FP8>(b1[1]);
        pair8(w8_bf16<FP8>(b1[0]), two ? hu : z, up);
      }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const uint32_t x2 = xp[m * np + q];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc[0][m][e] = dot2(x2, wp[e], acc[0][m][e]);
        if constexpr (SWIGLU) acc[1][m][e] = dot2(x2, up[e], acc[1][m][e]);
      }
    }
  }
  // the 8 k lanes of a chunk: lanes 8j .. 8j + 7 of the wave, a fixed tree
#pragma unroll
  for (int w = 0; w < (SWIGLU ? 2 : 1); ++w) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float v = acc[w][m][e];
        v += __shfl_xor(v, 1, 64);
        v += __shfl_xor(v, 2, 64);
        v += __shfl_xor(v, 4, 64);
        acc[w][m][e] = v;
      }
    }
  }
  if (kl == 0 && incol) {
#pragma unroll
    for (int w = 0; w < (SWIGLU ? 2 : 1); ++w) {
      float *P = a.ws + (int64_t)w * a.ksplit * a.M * a.N + ((int64_t)ks * a.M) * a.N + col;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m < M) {
          float4 *p = reinterpret_cast<float4 *>(P + m * a.N);
          p[0] = make_float4(acc[w][m][0], acc[w][m][1], acc[w][m][2], acc[w][m][3]);
          p[1] = make_float4(acc[w][m][4], acc[w][m][5], acc[w][m][6], acc[w][m][7]);
        }
      }
    }
  }
}

template <bool FP8, bool SWIGLU, int MT>
__device__ __forceinline__ void gemv_nt_body(const GemvArgs &a) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[GV_MAX_M * GV_MAX_KC];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ks = blockIdx.x % a.ksplit;
  const int64_t nb = (int64_t)(blockIdx.x / a.ksplit) * (4 * NT_ROWS) + wave * NT_ROWS;
  const int64_t k0 = (int64_t)ks * a.kc;
  stage_a<MT>(a, xs, k0);
  __syncthreads();

  constexpr int CK = FP8 ? 16 : 8;  // k per 16-byte chunk
  const int M = (int)a.M;
  float acc[SWIGLU ? 2 : 1][MT][NT_ROWS];
#pragma unroll
  for (int w = 0; w < (SWIGLU ? 2 : 1); ++w)
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < NT_ROWS; ++r) acc[w][m][r] = 0.f;
  const int kend = (int)min((int64_t)a.kc, a.K - k0);  // a multiple of CK
  for (int kk = lane * CK; kk < kend; kk += 64 * CK) {
    // this chunk of every row first (NT_ROWS loads per weight in flight)
    uint4 raw0[NT_ROWS], raw1[NT_ROWS];
#pragma unroll
    for (int r = 0; r < NT_ROWS; ++r) {
      const int64_t n = min(nb + r, a.N - 1);  // rows past N: loaded, never stored
      const int64_t off = (n * a.ldb + k0 + kk) * (FP8 ? 1 : 2);
      raw0[r] = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint8_t *>(a.B0) + off);
      if constexpr (SWIGLU) raw1[r] = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint8_t *>(a.B1) + off);
    }
#pragma unroll
    for (int h = 0; h < CK / 8; ++h) {
      uint4 xw[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) xw[m] = *reinterpret_cast<const uint4 *>(xs + m * a.kc + kk + 8 * h);
#pragma unroll
      for (int r = 0; r < NT_ROWS; ++r) {
        uint4 f, fu;
        if constexpr (FP8) {
          f = e4m3x8_to_bf16x8(h ? make_uint2(raw0[r].z, raw0[r].w) : make_uint2(raw0[r].x, raw0[r].y));
          if constexpr (SWIGLU)
            fu = e4m3x8_to_bf16x8(h ? make_uint2(raw1[r].z, raw1[r].w) : make_uint2(raw1[r].x, raw1[r].y));
        } else {
          f = raw0[r];
          if constexpr (SWIGLU) fu = raw1[r];
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          // consecutive k pair up in each word of both operands
          acc[0][m][r] = dot2(xw[m].x, f.x, acc[0][m][r]);
          acc[0][m][r] = dot2(xw[m].y, f.y, acc[0][m][r]);
          acc[0][m][r] = dot2(xw[m].z, f.z, acc[0][m][r]);
          acc[0][m][r] = dot2(xw[m].w, f.w, acc[0][m][r]);
          if constexpr (SWIGLU) {
            acc[1][m][r] = dot2(xw[m].x, fu.x, acc[1][m][r]);
            acc[1][m][r] = dot2(xw[m].y, fu.y, acc[1][m][r]);
            acc[1][m][r] = dot2(xw[m].z, fu.z, acc[1][m][r]);
            acc[1][m][r] = dot2(xw[m].w, fu.w, acc[1][m][r]);
          }
        }
      }
    }
  }
  // the 64 lanes: a fixed shuffle tree
#pragma unroll
  for (int w = 0; w < (SWIGLU ? 2 : 1); ++w)
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
      for (int r = 0; r < NT_ROWS; ++r) {
        float v = acc[w][m][r];
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
        acc[w][m][r] = v;
      }
    }
  if (lane == 0) {
#pragma unroll
    for (int w = 0; w < (SWIGLU ? 2 : 1); ++w) {
      float *P = a.ws + (int64_t)w * a.ksplit * a.M * a.N + ((int64_t)ks * a.M) * a.N;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
#pragma unroll
        for (int r = 0; r < NT_ROWS; ++r)
          if (m < M && nb + r < a.N) P[m * a.N + nb + r] = acc[w][m][r];
      }
    }
  }
}

#define NK_GEMV_M(layout, wt, FP8, MT)                                                               \
  extern "C" __global__ __launch_bounds__(256) void nk_gemv_##layout##_##wt##_m##MT(GemvArgs a) {    \
    gemv_##layout##_body<FP8, false, MT>(a);                                                          \
  }                                                                                                   \
  extern "C" __global__ __launch_bounds__(256) void nk_gemv_##layout##_##wt##_swiglu_m##MT(GemvArgs a) { \
    gemv_##layout##_body<FP8, true, MT>(a);                                                           \
  }
#define NK_GEMV(layout, wt, FP8) NK_GEMV_M(layout, wt, FP8, 1) NK_GEMV_M(layout, wt, FP8, 4) NK_GEMV_M(layout, wt, FP8, 8)
NK_GEMV(nn, bf16, false)
NK_GEMV(nn, e4m3, true)
NK_GEMV(nt, bf16, false)
NK_GEMV(nt, e4m3, true)

// The splits added, then the GEMM's epilogue.  A workgroup serves 64
// consecutive outputs (flattened m * N + n); wave j adds splits j, j + 4,
// j + 8, ... in order, each of its loads covering the 64 outputs (256
// contiguous bytes) and all of them issued before the first add (16 at a
// time); wave 0 then combines the four wave sums as (s0 + s1) + (s2 + s3).
// A fixed order, one or two memory round trips for up to 64 splits.
template <typename TC, bool SWIGLU>
__device__ __forceinline__ void gemv_out_body(const GemvArgs &a) {
  __shared__ float red[2][4][64];
  const int lane = threadIdx.x & 63, j = threadIdx.x >> 6;
  const int64_t plane = a.M * a.N;
  const int64_t o = (int64_t)blockIdx.x * 64 + lane;
  const bool live = o < plane;
  const int64_t i = live ? o : 0;  // dead lanes read output 0, store nothing
  float g = 0.f, u = 0.f;
  for (int s0 = j; s0 < a.ksplit; s0 += 64) {
    float x[16], y[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int s = min(s0 + 4 * q, a.ksplit - 1);
      x[q] = a.ws[s * plane + i];
      y[q] = SWIGLU ? a.ws[(a.ksplit + s) * plane + i] : 0.f;
    }
#pragma unroll
    for (int q = 0; q < 16; ++q)
      if (s0 + 4 * q < a.ksplit) {
        g += x[q];
        if constexpr (SWIGLU) u += y[q];
      }
  }
  red[0][j][lane] = g;
  if constexpr (SWIGLU) red[1][j][lane] = u;
  __syncthreads();
  if (j != 0 || !live) return;
  g = (red[0][0][lane] + red[0][1][lane]) + (red[0][2][lane] + red[0][3][lane]);
  if constexpr (SWIGLU) u = (red[1][0][lane] + red[1][1][lane]) + (red[1][2][lane] + red[1][3][lane]);
  const int64_t m = i / a.N, n = i % a.N;
  float v;
  if constexpr (SWIGLU) {
    if (a.flags & GEMM_SCALE) {
      g *= a.scale0[n];
      u *= a.scale1[n];
    }
    // silu(g) = g / (1 + exp(-g)) from the hardware 2^x and reciprocal, as
    // the GEMM's epilogue computes it
    const float ex = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
    v = g * __builtin_amdgcn_rcpf(1.0f + ex) * u;
  } else {
    float prod = (a.flags & GEMM_SCALE) ? g * a.scale0[n] : g;
    const float bias = (a.flags & GEMM_BIAS) ? bf16_to_f32(a.bias[n]) : 0.f;
    if (a.flags & GEMM_RND_BIAS) prod = bf16_to_f32(f32_to_bf16(prod));
    v = prod + bias;
    if (a.flags & GEMM_RND_RESID) v = bf16_to_f32(f32_to_bf16(v));
    if (a.flags & GEMM_RESID) v += Elt<TC>::load(reinterpret_cast<const TC *>(a.resid), m * a.ldc + n);
  }
  Elt<TC>::store(reinterpret_cast<TC *>(a.C), m * a.ldc + n, v);
}

extern "C" __global__ __launch_bounds__(256) void nk_gemv_out_bf16(GemvArgs a) { gemv_out_body<bf16, false>(a); }
extern "C" __global__ __launch_bounds__(256) void nk_gemv_out_f32(GemvArgs a) { gemv_out_body<float, false>(a); }
extern "C" __global__ __launch_bounds__(256) void nk_gemv_out_bf16_swiglu(GemvArgs a) {
  gemv_out_body<bf16, true>(a);
}

// ---------------------------------------------------------------------------
// MFMA form of the NN partial sums (bf16 K x N weights) for up to 16 MT rows.
// The VALU kernel above spends a multiply-add per row on every weight; here
// the rows ride on 16x16x32 MFMAs (A: 16 rows x 32 k, zero rows past M) and
// the weights are streamed once:
//  * a workgroup (4 waves) owns 256 columns and one K range of kc (a
//    multiple of 32, at most GK_MAX_KC / MT); wave w owns columns 64 w..64 w + 63
//    (four 16-column tiles);
//  * the weights of the range move global -> LDS by DMA in stages of 32 k
//    rows x 256 columns (16 KiB: two column halves [32 k][128 n] of 256-byte
//    rows, 16-byte chunk c of row k at slot c ^ ((k & 3) << 2)) through a
//    ring of three slots, two stages ahead of the one read (two workgroups
//    fit a CU);
//    B fragments come out transposed (ds_read_b64_tr_b16: lane (g, i) reads
//    k rows 8 g + 4 s + i / 4 at columns c + 4 (i % 4), and receives k
//    8 g + 4 s .. + 3 of column c + i);
//  * A's rows of the range move into LDS by DMA once, rows of kc + 8
//    elements (an odd number of 16-byte chunks, so the 16 rows of a fragment
//    read fall on 16 distinct bank groups), zeros past M and past the range.
// Rows past the range end, and columns past N, are moves out of the
// resource's range: zeros, no memory read.  The partial sums go to the
// workspace as in nk_gemv_nn_*: P[split][m][n], rows m < M.  SwiGLU form
// (_swiglu): a workgroup owns 128 output columns; a stage holds those
// columns of the gate weights in its first half and of the up weights in
// its second, so waves 0-1 sum gate columns and waves 2-3 up columns, into
// the two sets of planes the SwiGLU reduction reads.
// ---------------------------------------------------------------------------
#define GK_MAX_KC 512

typedef short gk_s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) gk_s16x4 gk_lds_s16x4;
typedef __bf16 gk_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 gk_bf16x4 __attribute__((ext_vector_type(4)));
typedef float gk_f32x4 __attribute__((ext_vector_type(4)));

template <int MT, bool SWIGLU>
__device__ __forceinline__ void gemv_mfma_nn_body(const GemvArgs &a) {
  constexpr int GK_STAGES = 3;
  constexpr int SB = 32 * 256 * 2;                                       // one stage
  constexpr int AB = ((16 * MT * (GK_MAX_KC / MT + 8) * 2 + 1023) / 1024) * 1024;  // A rows, whole 1 KiB moves
  __shared__ __attribute__((aligned(1024))) uint8_t ring[GK_STAGES * SB];
  __shared__ __attribute__((aligned(1024))) uint8_t as[AB];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g4 = lane >> 4;
  const int ks = blockIdx.x % a.ksplit;
  const int64_t n0 = (int64_t)(blockIdx.x / a.ksplit) * (SWIGLU ? 128 : 256);
  const int64_t k0 = (int64_t)ks * a.kc;
  const int kend = (int)min((int64_t)a.kc, a.K - k0);  // a multiple of 8
  const int nst = (kend + 31) >> 5;                    // stages of this range
  const int cpr = a.kc >> 3;                           // 16-byte chunks per A row

  // A: slot s of the row-padded layout holds row s / (cpr + 1), chunk
  // s % (cpr + 1) (the last chunk of a row is padding)
  {
    const i32x4_t ra = rsrc_words(a.A, a.M * a.lda * 2);
    const int nslot = 16 * MT * (cpr + 1);
    for (int j = wave; j * 64 < nslot; j += 4) {
      const int s = j * 64 + lane;
      const int r = s / (cpr + 1), c = s % (cpr + 1);
      const bool in = s < nslot && c < cpr && 8 * c < kend && r < a.M;
      dma16_asm(ra, lds_addr(as) + j * 1024, in ? (uint32_t)((r * a.lda + k0 + 8 * c) * 2) : 0x80000000u);
    }
  }
  // B stage t into ring slot t % GK_STAGES: block b = wave + 4 j (j < 4)
  // covers k rows 4 (b % 8) + lane / 16 of column half b / 8
  const i32x4_t rb = rsrc_words(reinterpret_cast<const uint16_t *>(a.B0) + k0 * a.ldb, (int64_t)kend * a.ldb * 2);
  const i32x4_t ru = rsrc_words(SWIGLU ? reinterpret_cast<const uint16_t *>(a.B1) + k0 * a.ldb : nullptr,
                                SWIGLU ? (int64_t)kend * a.ldb * 2 : 0);
  uint32_t boff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int b = wave + 4 * j;
    const int kr = 4 * (b & 7) + g4;
    const int lc = l16 ^ ((kr & 3) << 2);
    const int64_t col = n0 + (SWIGLU ? 0 : 128 * (b >> 3)) + 8 * lc;
    boff[j] = col < a.N ? (uint32_t)((kr * a.ldb + col) * 2) : 0x80000000u;
  }
  const uint32_t tstep = (uint32_t)(32 * a.ldb * 2);
  auto stage = [&](int t) __attribute__((always_inline)) {
    const uint32_t base = lds_addr(ring) + (t % GK_STAGES) * SB;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int b = wave + 4 * j;
      // stages past the range read nothing (every offset out of range)
      dma16_asm((SWIGLU && (b >> 3)) ? ru : rb, base + b * 1024,
                t < nst && boff[j] != 0x80000000u ? boff[j] + t * tstep : 0x80000000u);
    }
  };
#pragma unroll
  for (int t = 0; t < GK_STAGES - 1; ++t) stage(t);

  // fragment offsets: B tile jt of this wave (columns 64 wave + 16 jt), A
  // tile mt (rows 16 mt + l16, chunk g4 of the stage's four)
  uint32_t bfo[4];
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) {
    const int br = 64 * wave + 16 * jt;
    const int nl = (br & 127) + 4 * (l16 & 3);
    const int k = 8 * g4 + (l16 >> 2);
    bfo[jt] = (br >> 7) * 8192 + k * 256 + (((nl >> 3) ^ ((k & 3) << 2)) << 4) + (nl & 7) * 2;
  }
  const uint32_t afo = (uint32_t)((l16 * (cpr + 1) + g4) * 16);

  gk_f32x4 acc[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[mt][jt][r] = 0.f;
  for (int t = 0; t < nst; ++t) {
    // stage t (and A) landed for this wave: only the GK_STAGES - 2 later
    // stages' moves may be outstanding; the barrier then covers every
    // wave's moves and every wave's reads of the slot refilled next
    __builtin_amdgcn_s_waitcnt(0x0F70 | (4 * (GK_STAGES - 2)));
    lds_barrier();
    stage(t + GK_STAGES - 1);
    const uint8_t *S = ring + (t % GK_STAGES) * SB;
    gk_bf16x8 bf[4], af[MT];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      const gk_s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((gk_lds_s16x4 *)(S + bfo[jt]));
      const gk_s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((gk_lds_s16x4 *)(S + bfo[jt] + 4 * 256));
      bf[jt] = __builtin_shufflevector(__builtin_bit_cast(gk_bf16x4, v0), __builtin_bit_cast(gk_bf16x4, v1), 0, 1,
                                       2, 3, 4, 5, 6, 7);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      af[mt] = *reinterpret_cast<const gk_bf16x8 *>(as + afo + (16 * mt * (cpr + 1) + 4 * t) * 16);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
        acc[mt][jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bf[jt], acc[mt][jt], 0, 0, 0);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): no move outlives the workgroup

  // D rows 16 mt + 4 g4 + r, column 64 wave + 16 jt + l16 (SwiGLU: column
  // 64 (wave % 2) + 16 jt + l16 of the gate or the up planes)
  float *P = a.ws + ((SWIGLU ? (int64_t)(wave >> 1) * a.ksplit : 0) + ks) * a.M * a.N;
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) {
    const int64_t n = n0 + 64 * (SWIGLU ? (wave & 1) : wave) + 16 * jt + l16;
    if (n < a.N) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * mt + 4 * g4 + r;
          if (m < a.M) P[m * a.N + n] = acc[mt][jt][r];
        }
    }
  }
}

extern "C" __global__ __launch_bounds__(256) void nk_gemv_mfma_nn_bf16_t1(GemvArgs a) {
  gemv_mfma_nn_body<1, false>(a);
}
extern "C" __global__ __launch_bounds__(256) void nk_gemv_mfma_nn_bf16_t2(GemvArgs a) {
  gemv_mfma_nn_body<2, false>(a);
}
extern "C" __global__ __launch_bounds__(256) void nk_gemv_mfma_nn_bf16_swiglu_t1(GemvArgs a) {
  gemv_mfma_nn_body<1, true>(a);
}
extern "C" __global__ __launch_bounds__(256) void nk_gemv_mfma_nn_bf16_swiglu_t2(GemvArgs a) {
  gemv_mfma_nn_body<2, true>(a);
}

// ---------------------------------------------------------------------------
// MFMA form of the NT partial sums (weights N x K, each row contiguous in k:
// bf16, or fp8 e4m3 decoded exactly to bf16) for up to 16 MT rows.  Every
// wave loads its B fragments straight from global memory into registers,
// and A's (16 rows x 32 k, L2-resident) the same way: no LDS and no
// barrier.  The K range goes in super-steps of 64 k in which lane (g, i)
// owns k 16g..16g+15 of column i's row (32 contiguous bytes of bf16, 16 of
// fp8, so the four lanes of a row read 128 / 64 contiguous bytes); the
// super-step's two 16x16x32 MFMAs take k 16g + 8s .. + 7 (s = 0, 1) in
// the fragment slots 8g..8g+7 of both operands, a permutation of the 64 k
// that A and B share.  PF super-steps are in flight.  A workgroup (4
// waves) owns 256 columns and one K range of kc (a multiple of 32); wave w
// owns columns 64w.. (four 16-column tiles).  The SwiGLU form owns 128
// columns: waves 0-1 read the gate rows, waves 2-3 the up rows, into the
// two sets of planes of the SwiGLU reduction.  Columns past N and k past the
// range are loads out of the resource's range (zeros, no memory read; fp8
// ranges end on a multiple of 16).  Partial sums as in nk_gemv_nt_*:
// P[split][m][n].
// ---------------------------------------------------------------------------
template <int MT, bool FP8, bool SWIGLU>
__device__ __forceinline__ void gemv_mfma_nt_body(const GemvArgs &a) {
  constexpr int ES = FP8 ? 1 : 2;       // weight element bytes
  constexpr int NB = FP8 ? 1 : 2;       // 16-byte weight loads per tile and super-step
  constexpr int PF = FP8 ? 4 : 2;       // super-steps in flight
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g4 = lane >> 4;
  const int ks = blockIdx.x % a.ksplit;
  const int64_t n0 = (int64_t)(blockIdx.x / a.ksplit) * (SWIGLU ? 128 : 256);
  const int64_t k0 = (int64_t)ks * a.kc;
  const int kend = (int)min((int64_t)a.kc, a.K - k0);  // a multiple of 8 (16 with fp8)
  const int nss = (kend + 63) >> 6;                    // super-steps
  const bool up = SWIGLU && wave >= 2;
  const int64_t nw = n0 + 64 * (SWIGLU ? (wave & 1) : wave);  // this wave's first column

  // byte offsets at super-step 0 (+ 64 elements per super-step); out of
  // range: 2^31
  const auto rb = buf_rsrc(up ? a.B1 : a.B0, (uint32_t)(a.N * a.ldb * ES));
  const auto ra = buf_rsrc(a.A, (uint32_t)(a.M * a.lda * 2));
  uint32_t boff[4], aoff[MT];
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) {
    const int64_t n = nw + 16 * jt + l16;
    boff[jt] = n < a.N ? (uint32_t)((n * a.ldb + k0 + 16 * g4) * ES) : 0x80000000u;
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + l16;
    aoff[mt] = m < a.M ? (uint32_t)((m * a.lda + k0 + 16 * g4) * 2) : 0x80000000u;
  }
  uint4 bq[PF][4][NB], aq[PF][MT][2];
  auto issue = [&](int u, int t) __attribute__((always_inline)) {
    // this lane's 8-k chunks of super-step t: 64 t + 16 g4 + 8 s < kend
    const int kb = 64 * t + 16 * g4;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int q = 0; q < NB; ++q) {
        const bool in = kb + 8 * q < kend && boff[jt] != 0x80000000u;
        bq[u][jt][q] = buf_ld16<false>(rb, in ? boff[jt] + 64 * t * ES + 16 * q : 0x80000000u);
      }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const bool in = kb + 8 * q < kend && aoff[mt] != 0x80000000u;
        aq[u][mt][q] = buf_ld16<false>(ra, in ? aoff[mt] + 128 * t + 16 * q : 0x80000000u);
      }
  };
#pragma unroll
  for (int u = 0; u < PF; ++u) issue(u, u);

  gk_f32x4 acc[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[mt][jt][r] = 0.f;
  for (int t0 = 0; t0 < nss; t0 += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      if (t0 + u < nss) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          gk_bf16x8 bf[4];
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) {
            if constexpr (FP8) {
              const uint4 w = bq[u][jt][0];
              bf[jt] = __builtin_bit_cast(gk_bf16x8, e4m3x8_to_bf16x8(s ? make_uint2(w.z, w.w) : make_uint2(w.x, w.y)));
            } else {
              bf[jt] = __builtin_bit_cast(gk_bf16x8, bq[u][jt][s]);
            }
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const gk_bf16x8 af = __builtin_bit_cast(gk_bf16x8, aq[u][mt][s]);
#pragma unroll
            for (int jt = 0; jt < 4; ++jt)
              acc[mt][jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf[jt], acc[mt][jt], 0, 0, 0);
          }
        }
      }
      issue(u, t0 + u + PF);  // past the range: loads of zeros, no memory read
    }
  }

  // D rows 16 mt + 4 g4 + r, column nw + 16 jt + l16
  float *P = a.ws + ((SWIGLU ? (int64_t)(wave >> 1) * a.ksplit : 0) + ks) * a.M * a.N;
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) {
    const int64_t n = nw + 16 * jt + l16;
    if (n < a.N) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * mt + 4 * g4 + r;
          if (m < a.M) P[m * a.N + n] = acc[mt][jt][r];
        }
    }
  }
}

#define NK_GEMV_MFMA_NT(wt, FP8)                                                                            \
  extern "C" __global__ __launch_bounds__(256) void nk_gemv_mfma_nt_##wt##_t1(GemvArgs a) {                 \
    gemv_mfma_nt_body<1, FP8, false>(a);                                                                    \
  }                                                                                                         \
  extern "C" __global__ __launch_bounds__(256) void nk_gemv_mfma_nt_##wt##_t2(GemvArgs a) {                 \
    gemv_mfma_nt_body<2, FP8, false>(a);                                                                    \
  }                                                                                                         \
  extern "C" __global__ __launch_bounds__(256) void nk_gemv_mfma_nt_##wt##_swiglu_t1(GemvArgs a) {          \
    gemv_mfma_nt_body<1, FP8, true>(a);                                                                     \
  }                                                                                                         \
  extern "C" __global__ __launch_bounds__(256) void nk_gemv_mfma_nt_##wt##_swiglu_t2(GemvArgs a) {          \
    gemv_mfma_nt_body<2, FP8, true>(a);                                                                     \
  }
NK_GEMV_MFMA_NT(bf16, false)
NK_GEMV_MFMA_NT(e4m3, true)
