// Causal grouped-query attention (flash-style, one pass) for gfx950.
//
//   o[b, s, h, :] = sum_t softmax_t(scale * q[b, s, h] . k[b, t, g(h)]  (t <= s)) v[b, t, g(h)]
//   g(h) = h / (Hq / Hkv)
//
// The NumPy composition it replaces is the attention block of the decoder
// kernels (tests/kernels/llama_decoder_dynamo.py:180-288,
// examples/models/qwen3/kernels/attention.py:109-140): np.repeat of the KV
// heads, q @ k^T scaled, causal mask added, softmax over keys, @ v.
//
// Work split: one workgroup (4 waves) per (b, h, block of 128 queries); each
// wave owns 32 queries.  The kernel computes S^T = K Q^T and O^T = V^T P^T
// with v_mfma_f32_32x32x16_bf16 so that every lane owns one query column:
// the running max / sum of the online softmax are lane-local (the two lane
// halves holding the same query combine with one xor-32 shuffle), and the
// P^T operand of the second product is taken straight from the S^T
// accumulators -- V^T is read in the matching permuted key order.
// Q fragments stay in registers; K tiles (64 keys x 128) and V^T tiles
// (128 x 64 keys, transposed in registers on the way in) are double-buffered
// in LDS.  Scores and softmax are fp32; P enters the second MFMA as bf16.
// Query blocks are issued longest-first (causal work grows with position).

#include "common.h"

using namespace nk;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define AQ 128  // queries per workgroup
#define AK 64   // keys per block
#define AD 128  // head dim

struct AttnArgs {
  const uint16_t *q;
  const uint16_t *k;
  const uint16_t *v;
  uint16_t *o;
  int64_t q_sb, q_ss, q_sh;  // element strides of q over (b, s, h); d contiguous
  int64_t k_sb, k_ss, k_sh;
  int64_t v_sb, v_ss, v_sh;
  int64_t o_sb, o_ss, o_sh;
  int32_t B, S, Hq, Hkv;
  float scale;
  int32_t causal;
};

__device__ __forceinline__ int koff(int row, int col) {  // K tile: rows of 128
  return row * AD + ((((col >> 3) ^ (row & 15))) << 3) + (col & 7);
}
__device__ __forceinline__ int voff(int row, int col) {  // V^T tile: rows of 64
  return row * AK + ((((col >> 3) ^ ((row >> 1) & 7))) << 3) + (col & 7);
}

extern "C" __global__ __launch_bounds__(256, 1) void nk_attention_causal_d128(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][AK * AD];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[2][AD * AK];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, lhi = lane >> 5;

  // block -> (b, h, query block), longest (last) query blocks first
  const int nqb = a.S / AQ;
  const int bid = blockIdx.x;
  const int qb = nqb - 1 - (bid % nqb);
  const int bh = bid / nqb;
  const int h = bh % a.Hq, b = bh / a.Hq;
  const int g = h / (a.Hq / a.Hkv);
  const int q0 = qb * AQ;

  const uint16_t *qp = a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh;
  const uint16_t *kp = a.k + (int64_t)b * a.k_sb + (int64_t)g * a.k_sh;
  const uint16_t *vp = a.v + (int64_t)b * a.v_sb + (int64_t)g * a.v_sh;
  uint16_t *op = a.o + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh;

  // this lane's query (column of S^T / O^T) and its Q fragments (B operand)
  const int qrow = q0 + wave * 32 + l32;
  bf16x8_t qf[AD / 16];
#pragma unroll
  for (int kk = 0; kk < AD / 16; ++kk)
    qf[kk] = *reinterpret_cast<const bf16x8_t *>(qp + (int64_t)qrow * a.q_ss + kk * 16 + lhi * 8);

  f32x16 acc_o[4];  // O^T tiles: rows d = dt*32 + ..., column = this query
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[t][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float sl2 = a.scale * 1.44269504088896340736f;  // scale * log2(e)

  const int kend = a.causal ? (q0 + AQ) : a.S;
  const int nkb = kend / AK;

  // staging: threads 0..127 transpose an 8 x 8 block of V, 128..255 load K
  uint4 stage[8];
  auto load_tile = [&](int kb) {
    const int t0 = kb * AK;
    if (tid < 128) {
      const int kblk = tid >> 4, dblk = tid & 15;  // 8 key blocks x 16 d blocks
#pragma unroll
      for (int j = 0; j < 8; ++j)
        stage[j] = *reinterpret_cast<const uint4 *>(vp + (int64_t)(t0 + kblk * 8 + j) * a.v_ss + dblk * 8);
    } else {
      const int t = tid - 128;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int c = t + 128 * i;
        const int row = c >> 4, col = (c & 15) * 8;
        stage[i] = *reinterpret_cast<const uint4 *>(kp + (int64_t)(t0 + row) * a.k_ss + col);
      }
    }
  };
  auto store_tile = [&](int buf) {
    if (tid < 128) {
      const int kblk = tid >> 4, dblk = tid & 15;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t w[4];
#pragma unroll
        for (int p = 0; p < 4; ++p)
          w[p] = h16_of(stage[2 * p], i) | (h16_of(stage[2 * p + 1], i) << 16);
        *reinterpret_cast<uint4 *>(Vt[buf] + voff(dblk * 8 + i, kblk * 8)) = make_uint4(w[0], w[1], w[2], w[3]);
      }
    } else {
      const int t = tid - 128;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int c = t + 128 * i;
        const int row = c >> 4, col = (c & 15) * 8;
        *reinterpret_cast<uint4 *>(Ks[buf] + koff(row, col)) = stage[i];
      }
    }
  };

  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
    if (kb + 1 < nkb) load_tile(kb + 1);

    // S^T = K Q^T for 64 keys: two 32 x 32 tiles (keys ktile*32 + ..)
    f32x16 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kt][r] = 0.f;
#pragma unroll
      for (int kk = 0; kk < AD / 16; ++kk) {
        bf16x8_t kf = *reinterpret_cast<const bf16x8_t *>(Ks[buf] + koff(kt * 32 + l32, kk * 16 + lhi * 8));
        s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], s[kt], 0, 0, 0);
      }
    }
    // scale (in log2 units), causal mask, block max
    const int key0 = kb * AK;
    float bmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = key0 + kt * 32 + (r >> 2) * 8 + lhi * 4 + (r & 3);
        float x = s[kt][r] * sl2;
        if (a.causal && key > qrow) x = -INFINITY;
        s[kt][r] = x;
        bmax = fmaxf(bmax, x);
      }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
    const float m_new = fmaxf(m_run, bmax);
    const float alpha = exp2f(m_run - m_new);  // 0 on the first block
    float bsum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = exp2f(s[kt][r] - m_new);
        s[kt][r] = p;
        bsum += p;
      }
    bsum += __shfl_xor(bsum, 32, 64);
    l_run = l_run * alpha + bsum;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_o[t][r] *= alpha;

    // O^T += V^T P^T; k-step j covers keys 16j..16j+15 in the permuted order
    // this lane's P values already have: {16j + 4*lhi + 0..3, 16j + 8 + 4*lhi + 0..3}
#pragma unroll
    for (int j = 0; j < AK / 16; ++j) {
      const int kt = j >> 1, g0 = (j & 1) * 8;
      bf16x8_t pf;
#pragma unroll
      for (int e = 0; e < 8; ++e) pf[e] = (__bf16)s[kt][g0 + e];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int d = t * 32 + l32;
        const bf16x4_t lo = *reinterpret_cast<const bf16x4_t *>(Vt[buf] + voff(d, 16 * j + 4 * lhi));
        const bf16x4_t hi = *reinterpret_cast<const bf16x4_t *>(Vt[buf] + voff(d, 16 * j + 8 + 4 * lhi));
        bf16x8_t vf;
        vf[0] = lo[0]; vf[1] = lo[1]; vf[2] = lo[2]; vf[3] = lo[3];
        vf[4] = hi[0]; vf[5] = hi[1]; vf[6] = hi[2]; vf[7] = hi[3];
        acc_o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, acc_o[t], 0, 0, 0);
      }
    }
    if (kb + 1 < nkb) store_tile(buf ^ 1);
    __syncthreads();
  }

  // normalise and store: lane holds d = t*32 + (r>>2)*8 + lhi*4 + (r&3) of its query
  const float inv_l = 1.0f / l_run;
  uint16_t *orow = op + (int64_t)qrow * a.o_ss;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      uint32_t w0 = (uint32_t)f32_to_bf16(acc_o[t][gq * 4 + 0] * inv_l) |
                    ((uint32_t)f32_to_bf16(acc_o[t][gq * 4 + 1] * inv_l) << 16);
      uint32_t w1 = (uint32_t)f32_to_bf16(acc_o[t][gq * 4 + 2] * inv_l) |
                    ((uint32_t)f32_to_bf16(acc_o[t][gq * 4 + 3] * inv_l) << 16);
      *reinterpret_cast<uint2 *>(orow + t * 32 + gq * 8 + lhi * 4) = make_uint2(w0, w1);
    }
}
