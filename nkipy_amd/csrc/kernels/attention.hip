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
// Work split: one workgroup of NW waves (4 or 8) per (b, h, block of 32 NW
// queries); each wave owns 32 queries; two workgroups share a CU.  The kernel computes
// S^T = K Q^T and O^T = V^T P^T with v_mfma_f32_32x32x16_bf16 so that every
// lane owns one query column: the running max / sum of the online softmax
// are lane-local (the two lane halves holding the same query combine with
// one xor-32 shuffle), and the P^T operand of the second product is taken
// straight from the S^T accumulators, whose key order the V^T fragments
// follow.
//
// Data movement: Q fragments stay in registers.  K and V tiles (64 keys x
// 128 d, d contiguous, exactly as they lie in memory) move global -> LDS by
// DMA (buffer_load ... lds), double-buffered.  The block loop is software
// pipelined: the step for block j runs the scores of block j + 1 on the
// MFMA pipe while the VALU does block j's softmax, so K runs one tile ahead
// of V.  K fragments are plain 16-byte LDS reads; V^T fragments come from
// ds_read_b64_tr_b16, which transposes 4 x 4 bf16 blocks across lanes on the
// way out of LDS.  Both tiles are XOR-swizzled so that these reads are bank
// conflict free.  Scores and the softmax are fp32 (running max kept stale
// up to a factor 2^8, so the O rescale is rare); P enters the second MFMA as
// bf16.  Causal masking is only evaluated on the final pair of blocks, and
// blocks entirely above a wave's diagonal are skipped.  Each XCD takes a
// contiguous range of (KV head, query head, query block) work items so one
// KV head's tiles are re-read from that XCD's L2; within a KV head the
// longest query blocks go first (causal work grows with position).

#include "common.h"

using namespace nk;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

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
  // score cast points of the *_xf kernels (ATT_* flags): the product rounded
  // to bf16, divided by `div` (rdiv = RN(1 / div)) instead of multiplied by
  // `scale`, the scaled score rounded to bf16
  float div, rdiv;
  int32_t flags;
  // the launches of the bf16 softmax (ATT_SOFTMAX_BF16) share per-query
  // statistics over chunks of ckb 32-key blocks (at most nch chunks per
  // row): for chunk c and row = (b * Hq + h) * S + query, the max score at
  // rowstat[c * B * Hq * S + row] and the sum of the weights at
  // rowstat[(nch + c) * B * Hq * S + row]
  float *rowstat;
  int32_t ckb, nch;
};
enum { ATT_RND_PROD = 1, ATT_RND_SCORE = 2, ATT_SOFTMAX_BF16 = 4, ATT_DIVIDE = 8 };

// K tile row (key) r: 16-byte chunk c stored at c ^ (r & 15): the 32 rows of
// a K fragment read hit 16 distinct bank slots (two per cycle's worth).
__device__ __forceinline__ int kswz(int r) { return r & 15; }
// V tile: chunk c of row r at c ^ 4 (r & 3): the 4 rows x 4 chunks of one
// transpose read land in 16 distinct slots.
__device__ __forceinline__ int vswz(int r) { return (r & 3) << 2; }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t *lds_block, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds_block, 16, off, 0, 0, 0);
}

__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

template <bool B> struct Flag {
  static constexpr bool value = B;
};

// NW waves (32 queries each) share one workgroup's K / V tiles: AQ = 32 NW
// queries per workgroup, two workgroups per CU (64 KiB of LDS each), so NW
// = 8 puts four waves on every SIMD (at most 128 registers each) and halves
// the K / V traffic per query.
// AKB keys per block (64, or 32: one 32 x 32 score tile, half the score
// registers and LDS, which lets three workgroups of four waves share a CU).
// PIPE: scores of block j + 1 computed while block j's softmax runs (two
// score sets live); without it a wave computes a block's scores, then its
// softmax, and the other waves on the SIMD fill the gaps.
template <int NW, int AKB, bool PIPE>
__device__ __forceinline__ void attention_causal_body(const AttnArgs &a) {
  constexpr int AQW = 32 * NW;  // queries per workgroup
  constexpr int AK = AKB;
  constexpr int KT = AK / 32;   // 32-key score tiles per block
  constexpr int TILE_BYTES = AK * AD * 2;
  __shared__ __attribute__((aligned(1024))) uint8_t K0[TILE_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t K1[TILE_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t V0[TILE_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t V1[TILE_BYTES];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31, lhi = lane >> 5;

  // Workgroup -> (b, KV head g, query head h, query block).  Workgroups are
  // dispatched round-robin over the 8 XCDs, so workgroup i runs on XCD i % 8;
  // giving each XCD a contiguous range of work items keeps the query heads
  // and blocks that share one K / V head on one XCD, whose L2 then serves
  // the K / V re-reads.  Within a KV head, the longest (last) query blocks
  // go first.
  const int nqb = a.S / AQW;
  const int rep = a.Hq / a.Hkv;
  const int per_kv = rep * nqb;
  const int nwg = a.B * a.Hkv * per_kv;  // the grid size
  int w = blockIdx.x;
  if ((nwg & 7) == 0) w = (w & 7) * (nwg >> 3) + (w >> 3);
  const int bg = w / per_kv, within = w % per_kv;
  const int qb = nqb - 1 - within / rep;
  const int g = bg % a.Hkv, b = bg / a.Hkv;
  const int h = g * rep + within % rep;
  const int q0 = qb * AQW;

  const uint16_t *qp = a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh;
  const uint16_t *kp = a.k + (int64_t)b * a.k_sb + (int64_t)g * a.k_sh;
  const uint16_t *vp = a.v + (int64_t)b * a.v_sb + (int64_t)g * a.v_sh;
  uint16_t *op = a.o + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kp, (int64_t)a.S * a.k_ss * 2);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vp, (int64_t)a.S * a.v_ss * 2);

  // this lane's query (column of S^T / O^T) and its Q fragments (B operand)
  const int wq0 = q0 + wave * 32;
  const int qrow = wq0 + l32;
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

  const int kend = a.causal ? (q0 + AQW) : a.S;
  const int nkb = kend / AK;

  // DMA plan: a tile is AK / 4 moves of 1 KiB (4 rows of 256 bytes); wave w
  // does the K and V moves m = NW j + w (rows 4 m ..).  The chunk a lane
  // fetches is the same for every j (the swizzles only see row & 15, and
  // 4 NW j is a multiple of 16).
  constexpr int NM = AK / 4 / NW;  // K (and V) moves per wave
  static_assert(NM >= 1 && NM * NW * 4 == AK, "moves per wave");
  const int kchunk = (lane & 15) ^ kswz(wave * 4 + (lane >> 4));
  const int vchunk = (lane & 15) ^ vswz(wave * 4 + (lane >> 4));
  // move j of this wave: rows 4 (NW j + wave) + lane / 16, i.e. the j = 0
  // source plus j times a uniform stride
  const int row0 = wave * 4 + (lane >> 4);
  const uint32_t kbase = (uint32_t)(((int64_t)row0 * a.k_ss + kchunk * 8) * 2);
  const uint32_t vbase = (uint32_t)(((int64_t)row0 * a.v_ss + vchunk * 8) * 2);
  const uint32_t kjs = (uint32_t)(NW * 4 * a.k_ss * 2), vjs = (uint32_t)(NW * 4 * a.v_ss * 2);
  auto load_k = [&](uint8_t *dst, int kb) {
    const uint32_t kst = (uint32_t)((int64_t)kb * AK * a.k_ss * 2);
#pragma unroll
    for (int j = 0; j < NM; ++j) dma16(rk, dst + (j * NW + wave) * 1024, kbase + j * kjs + kst);
  };
  auto load_v = [&](uint8_t *dst, int kb) {
    const uint32_t vst = (uint32_t)((int64_t)kb * AK * a.v_ss * 2);
#pragma unroll
    for (int j = 0; j < NM; ++j) dma16(rv, dst + (j * NW + wave) * 1024, vbase + j * vjs + vst);
  };

  // Per-lane LDS byte offsets (the swizzles only see lane bits).
  // K fragment (row kt*32 + l32, chunk 2 kk + lhi): kt*8192 + koff(kk), with
  // chunk (2 kk + lhi) ^ (l32 & 15) = (2 kk ^ (l32 & 14)) + (lhi ^ (l32 & 1)):
  // one lane base plus kk * 32 XOR a lane constant (no table of offsets).
  const int klb = l32 * 256 + ((lhi ^ (l32 & 1)) << 4);
  const int kx = (l32 & 14) << 4;
  auto koff = [&](int kk) __attribute__((always_inline)) { return klb + ((kk << 5) ^ kx); };
  // V^T transpose read (group g = lane/16, i = lane%16): source row
  // 16 j + 8 si + 4 (g/2) + i/4, columns dt*32 + 16 (g%2) + 4 (i%4):
  // (16 j + 8 si) * 256 + voff(dt).
  int vlb, vx;
  {
    const int grp = lane >> 4, gi = lane & 15;
    const int c0 = (grp & 1) * 2 + ((gi & 3) >> 1), vsh = (gi >> 2) & 3;
    vlb = (4 * (grp >> 1) + (gi >> 2)) * 256 + (c0 << 4) + (gi & 1) * 8;
    vx = vsh << 6;
  }
  auto voff = [&](int dt) __attribute__((always_inline)) { return vlb + ((dt << 6) ^ vx); };

  // S^T = K Q^T for one 64-key block (keys kt*32 + row, this lane's query)
  auto qk = [&](const uint8_t *Kt, f32x16 (&s)[KT]) __attribute__((always_inline)) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kt][r] = 0.f;
#pragma unroll
      for (int kk = 0; kk < AD / 16; ++kk) {
        const bf16x8_t kf = *reinterpret_cast<const bf16x8_t *>(Kt + kt * 8192 + koff(kk));
        s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], s[kt], 0, 0, 0);
      }
    }
  };

  // Online softmax of one block's scores and O^T += V^T P^T.  DIAG blocks
  // are the final pair of a row of blocks: under a causal mask they may
  // cross the diagonal of this wave's queries; every other block lies below
  // it for all four waves and runs without mask code.
  auto finish = [&](f32x16 (&s)[KT], const uint8_t *Vt, int key0, auto diag_flag) __attribute__((always_inline)) {
    constexpr bool DIAG = decltype(diag_flag)::value;
    // block max of the raw scores (the scale is positive, so it commutes
    // with the max), as a tree
    float mx[4 * KT];
#pragma unroll
    for (int i = 0; i < 4 * KT; ++i) {
      if constexpr (DIAG) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int kt = i >> 2, r = (i & 3) * 4 + e;
          const int key = key0 + kt * 32 + (r >> 2) * 8 + lhi * 4 + (r & 3);
          if (a.causal && key > qrow) s[kt][r] = -INFINITY;
        }
      }
      const int kt = i >> 2, r0 = (i & 3) * 4;
      mx[i] = fmaxf(fmaxf(s[kt][r0], s[kt][r0 + 1]), fmaxf(s[kt][r0 + 2], s[kt][r0 + 3]));
    }
    float bmax = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
    if constexpr (KT == 2) bmax = fmaxf(bmax, fmaxf(fmaxf(mx[4], mx[5]), fmaxf(mx[6], mx[7])));
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
    // Running max m_run in log2 units, kept stale: it moves only when some
    // row's block max exceeds it by more than 8, so every P stays <= 2^8 and
    // the O rescale runs on a few blocks per row instead of all of them.  The
    // first block (key 0, seen by every row) always moves it from -inf.
    const float m_blk = bmax * sl2;
    const bool moved = __any(m_blk > m_run + 8.0f);
    const float m_new = moved ? fmaxf(m_run, m_blk) : m_run;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first block, 1 if unmoved
    m_run = m_new;
    float ps[AK / 16];
#pragma unroll
    for (int j = 0; j < AK / 16; ++j) ps[j] = 0.f;
    bf16x8_t pf[AK / 16];
#pragma unroll
    for (int j = 0; j < AK / 16; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int kt = j >> 1, r = (j & 1) * 8 + e;
        const float p = __builtin_amdgcn_exp2f(fmaf(s[kt][r], sl2, -m_new));
        ps[j] += p;
        pf[j][e] = (__bf16)p;
      }
    float bsum = ps[0] + ps[1];
    if constexpr (KT == 2) bsum = bsum + (ps[2] + ps[3]);
    bsum += __shfl_xor(bsum, 32, 64);
    l_run = fmaf(l_run, alpha, bsum);
    if (moved) {
#pragma unroll
      for (int t2 = 0; t2 < 4; ++t2)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[t2][r] *= alpha;
    }
    // O^T += V^T P^T.  Step j covers 16 keys; this lane's P values (S^T rows)
    // are keys 16 j + 4 lhi + {0..3} and 16 j + 8 + 4 lhi + {0..3}, which is
    // the order of the two transpose reads below (source row 16 j + 8 si +
    // 4 (g/2) + i/4; output lane i of group g gets column dt*32 + 16 (g%2) + i
    // for 4 consecutive keys).
#pragma unroll
    for (int j = 0; j < AK / 16; ++j) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        s16x4 v[2];
#pragma unroll
        for (int si = 0; si < 2; ++si)
          v[si] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4 *)(Vt + (16 * j + 8 * si) * 256 + voff(dt)));
        const bf16x8_t vf = __builtin_shufflevector(__builtin_bit_cast(bf16x4_t, v[0]),
                                                    __builtin_bit_cast(bf16x4_t, v[1]), 0, 1, 2, 3, 4, 5, 6, 7);
        acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[j], acc_o[dt], 0, 0, 0);
      }
    }
  };

  // Software pipeline over blocks: block j's K tile sits in K[j & 1] and its
  // V tile in V[j & 1]; the step for block j computes the scores of block
  // j + 1 while it runs block j's softmax and PV, and streams in K_{j+2} and
  // V_{j+1} meanwhile (K runs one tile ahead of V).  The buffers a step
  // overwrites were last read before the previous step's barrier.  Loads
  // past the blocks a workgroup needs read in-range rows it ignores, or zeros
  // past the end of the sequence.
  // Blocks 0 .. nd-1 lie below the diagonal of every wave (causal: the keys
  // before the workgroup's first query); the last blocks are the
  // diagonal blocks (AQW / AK of them), masked per key and skipped by the
  // waves whose queries all precede them (every wave still takes part in the loads and
  // barriers).  nd and the number of diagonal blocks are even.
  constexpr int NDIAG = AQW / AK;  // diagonal blocks (even)
  static_assert(NDIAG % 2 == 0, "diagonal blocks come in pairs");
  const int nd = a.causal ? q0 / AK : nkb - NDIAG;
  auto needed = [&](int j) { return !a.causal || j * AK <= wq0 + 31; };
  if constexpr (!PIPE) {
    f32x16 sc[KT];
    auto step1 = [&](int j, const uint8_t *kc, const uint8_t *vc, uint8_t *kn, uint8_t *vn, auto diag_flag)
        __attribute__((always_inline)) {
      constexpr bool DIAG = decltype(diag_flag)::value;
      load_k(kn, j + 1);
      load_v(vn, j + 1);
      if (!DIAG || needed(j)) {
        qk(kc, sc);
        finish(sc, vc, j * AK, diag_flag);
      }
      wait_vmem();
      __syncthreads();
    };
    load_k(K0, 0);
    load_v(V0, 0);
    wait_vmem();
    __syncthreads();
    for (int kb = 0; kb < nd; kb += 2) {
      step1(kb, K0, V0, K1, V1, Flag<false>{});
      step1(kb + 1, K1, V1, K0, V0, Flag<false>{});
    }
#pragma unroll
    for (int t = 0; t < NDIAG; t += 2) {
      step1(nd + t, K0, V0, K1, V1, Flag<true>{});
      step1(nd + t + 1, K1, V1, K0, V0, Flag<true>{});
    }
  } else {
  f32x16 sa[KT], sb[KT];
  auto step = [&](int j, f32x16 (&cur)[KT], f32x16 (&nxt)[KT], uint8_t *kdst, uint8_t *vdst, const uint8_t *knext,
                  const uint8_t *vcur, auto diag_flag) __attribute__((always_inline)) {
    constexpr bool DIAG = decltype(diag_flag)::value;
    load_k(kdst, j + 2);
    load_v(vdst, j + 1);
    if (!DIAG || (j + 1 < nkb && needed(j + 1))) qk(knext, nxt);
    if (!DIAG || needed(j)) finish(cur, vcur, j * AK, diag_flag);
    wait_vmem();
    __syncthreads();
  };
  load_k(K0, 0);
  load_v(V0, 0);
  load_k(K1, 1);  // nkb >= 2: S and the causal extent are multiples of 128 keys
  wait_vmem();
  __syncthreads();
  qk(K0, sa);
  __syncthreads();
  for (int kb = 0; kb < nd; kb += 2) {
    step(kb, sa, sb, K0, V1, K1, V0, Flag<false>{});
    step(kb + 1, sb, sa, K1, V0, K0, V1, Flag<false>{});
  }
#pragma unroll
  for (int t = 0; t < NDIAG; t += 2) {
    step(nd + t, sa, sb, K0, V1, K1, V0, Flag<true>{});
    step(nd + t + 1, sb, sa, K1, V0, K0, V1, Flag<true>{});
  }
  }

  // normalise and store: lane holds d = t*32 + (r>>2)*8 + lhi*4 + (r&3) of its query
  const float inv_l = 1.0f / l_run;
  uint16_t *orow = op + (int64_t)qrow * a.o_ss;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const uint32_t w0 = pack_bf16x2(acc_o[t][gq * 4 + 0] * inv_l, acc_o[t][gq * 4 + 1] * inv_l);
      const uint32_t w1 = pack_bf16x2(acc_o[t][gq * 4 + 2] * inv_l, acc_o[t][gq * 4 + 3] * inv_l);
      *reinterpret_cast<uint2 *>(orow + t * 32 + gq * 8 + lhi * 4) = make_uint2(w0, w1);
    }
}

// ---------------------------------------------------------------------------
// Software-pipelined variant.  Same operand layouts as above (S^T = K Q^T and
// O^T = V^T P^T on 32x32x16 MFMAs, one query column per lane, the same K / V
// swizzles), 32-key blocks, and rings of four LDS slots for K and for V.
//
// Iteration j issues, in one basic block, the score MFMAs of block j + 1 and
// the P V MFMAs of block j - 1, interleaved with the softmax of block j on
// the VALU: the matrix pipe stays fed while the wave evaluates its
// exponentials, instead of the two phases following each other.  K of block
// j + 4 and V of block j + 2 move into the slots freed by the previous
// iteration, so each DMA has three iterations to land; one barrier per block.
//
// Softmax offset: p = 2^(s c - m) with c = scale log2(e) and a per-query
// offset m that is not the running max.  m starts at the first block's max
// and is raised (O and l rescaled, the block recomputed) only when some lane's
// sum over its 16 scores of a block exceeds 2^16; otherwise no max is taken,
// so the common block costs one fma, one exp, one add and half a convert per
// score.  Every p stays below 2^16: nothing overflows, and since the output
// is a ratio of sums of the same p, the offset does not change it.
// ---------------------------------------------------------------------------
template <int N> struct SlotTag {
  static constexpr int value = N;
};


// the score cast points of the flags (uniform branches: every lane takes the
// same ones; the quotient of a finite score needs no infinity fallback in
// the block form)
__device__ __forceinline__ float cast_score(const AttnArgs &a, float x) {
  if (a.flags & ATT_RND_PROD) x = bf16_to_f32(f32_to_bf16(x));
  x = (a.flags & ATT_DIVIDE) ? div_rn(x, a.div, a.rdiv) : x * a.scale;
  if (a.flags & ATT_RND_SCORE) x = bf16_to_f32(f32_to_bf16(x));
  return x;
}
__device__ __forceinline__ void round_bf16x2(float &x0, float &x1);
__device__ __forceinline__ void round_block(f32x16 &s) {
#pragma unroll
  for (int r = 0; r < 16; r += 2) {
    float x0 = s[r], x1 = s[r + 1];
    round_bf16x2(x0, x1);
    s[r] = x0;
    s[r + 1] = x1;
  }
}
__device__ __forceinline__ void cast_block(const AttnArgs &a, f32x16 &s) {
  if (a.flags & ATT_RND_PROD) round_block(s);
  if (a.flags & ATT_DIVIDE) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = div_rn_finite(s[r], a.div, a.rdiv);
  } else {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] *= a.scale;
  }
  if (a.flags & ATT_RND_SCORE) round_block(s);
}
// query block qb's key chunks (bf16 softmax statistics)
__device__ __forceinline__ int stat_chunks(const AttnArgs &a, int qb) {
  const int nb = a.causal ? (qb + 1) * 4 : a.S / 32;
  return (nb + a.ckb - 1) / a.ckb;
}

// x0, x1 rounded to bf16 (round to nearest even) with one packed
// conversion.  The compiler splits a packed conversion whose halves are
// used apart into two single ones; an empty asm that takes the packed word
// keeps it whole.  (The conversion itself stays the compiler's, so its
// hazard checks cover it: an instruction written in asm that reads a
// v_exp_f32 result gets no wait state from the compiler.)
__device__ __forceinline__ void round_bf16x2(float &x0, float &x1) {
  uint32_t w = pack_bf16x2(x0, x1);
  asm("" : "+v"(w));
  x0 = __uint_as_float(w << 16);
  x1 = __uint_as_float(w & 0xffff0000u);
}

// XF: each score first takes the cast points the traced code applies
// before its softmax (the Qwen3 prefill form, examples/models/qwen3/kernels/
// attention.py:119-120: (q @ k^T) in bf16, divided by sqrt(d) in fp32, cast
// to bf16), then enters the softmax with a unit scale.
//
// SMX selects the softmax: false, online in fp32 with the offset described
// above; true, the bf16 softmax of the traced code (examples/models/qwen3/
// kernels/softmax.py:4-6 on bf16 scores) with every cast point, given each
// query's max score m and weight sum l from the row statistics kernels
// below: the weights p = bf16(e / l) with e = bf16(exp(bf16(s - m))) are
// the P V operand, and o = bf16(sum p v): the traced code's arithmetic, up
// to the order of the fp32 sums.  bf16(e / l) is formed as bf16(e RN(1 / l)):
// e and l have 8-bit significands, so e / l is never a bf16 rounding
// midpoint (a midpoint times l has a set bit below e's last) and lies at
// least 2^-17 (relative) from one, beyond the 2^-23 the product can stray
// from the correctly rounded quotient: both round to the same bf16 value.
template <int NW, bool XF = false, bool SMX = false>
__device__ __forceinline__ void attention_sp_body(const AttnArgs &a) {
  static_assert(!SMX || XF, "the bf16 softmax follows the score cast points");
  constexpr int AQW = 32 * NW;  // queries per workgroup
  constexpr int TB = 32 * AD * 2;  // one 32-key K or V tile
  // one array per operand: a slot is a constant offset, so one address
  // register per fragment serves all four slots
  __shared__ __attribute__((aligned(1024))) uint8_t KR[4 * TB];
  __shared__ __attribute__((aligned(1024))) uint8_t VR[4 * TB];
  auto kslot = [&](auto t) __attribute__((always_inline)) -> uint8_t * {
    return KR + (decltype(t)::value & 3) * TB;
  };
  auto vslot = [&](auto t) __attribute__((always_inline)) -> uint8_t * {
    return VR + (decltype(t)::value & 3) * TB;
  };

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31, lhi = lane >> 5;

  // work item order as in attention_causal_body: contiguous ranges per XCD,
  // longest query blocks of a KV head first
  const int nqb = a.S / AQW;
  const int rep = a.Hq / a.Hkv;
  const int per_kv = rep * nqb;
  const int nwg = a.B * a.Hkv * per_kv;
  int w = blockIdx.x;
  if ((nwg & 7) == 0) w = (w & 7) * (nwg >> 3) + (w >> 3);
  const int bg = w / per_kv, within = w % per_kv;
  const int qb = nqb - 1 - within / rep;
  const int g = bg % a.Hkv, b = bg / a.Hkv;
  const int h = g * rep + within % rep;
  const int q0 = qb * AQW;

  const uint16_t *qp = a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh;
  const uint16_t *kp = a.k + (int64_t)b * a.k_sb + (int64_t)g * a.k_sh;
  const uint16_t *vp = a.v + (int64_t)b * a.v_sb + (int64_t)g * a.v_sh;
  uint16_t *op = a.o + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh;
  const i32x4_t rk = rsrc_words(kp, (int64_t)a.S * a.k_ss * 2);
  const i32x4_t rv = rsrc_words(vp, (int64_t)a.S * a.v_ss * 2);
  // a resource of no bytes: moves of blocks past the workgroup's last write
  // zeros and read no memory
  const i32x4_t rnone = rsrc_words(kp, 0);

  const int wq0 = q0 + wave * 32;
  const int qrow = wq0 + l32;
  // SMX: this query's max score, bf16 weight sum and RN(1 / sum), from the
  // statistics of its query block's key chunks (the sums added in chunk
  // order)
  float mx = 0.f, lb = 1.f, rlb = 1.f;
  if constexpr (SMX) {
    const int64_t nq = (int64_t)a.B * a.Hq * a.S;
    const float *st = a.rowstat + ((int64_t)b * a.Hq + h) * a.S + qrow;
    const int nc = stat_chunks(a, qb);
    mx = st[0];
    float tot = st[a.nch * nq];
    for (int c = 1; c < nc; ++c) {
      mx = fmaxf(mx, st[c * nq]);
      tot += st[(a.nch + c) * nq];
    }
    lb = bf16_to_f32(f32_to_bf16(tot));
    rlb = __frcp_rn(lb);
  }
  bf16x8_t qf[AD / 16];
#pragma unroll
  for (int kk = 0; kk < AD / 16; ++kk)
    qf[kk] = *reinterpret_cast<const bf16x8_t *>(qp + (int64_t)qrow * a.q_ss + kk * 16 + lhi * 8);

  f32x16 acc_o[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[t][r] = 0.f;
  // m: the softmax offset in log2 units, finite so that masked scores (-inf)
  // give p = 0 and the first block (p = inf) always takes the recompute path
  float m_run = -1e30f, l_run = 0.f;
  const float sl2 = XF ? 1.44269504088896340736f : a.scale * 1.44269504088896340736f;

  // key blocks: the workgroup's (the last wave's causal extent) and this wave's
  const int nb_wg = a.causal ? (q0 + AQW) / 32 : a.S / 32;
  const int nb_w = a.causal ? wq0 / 32 + 1 : a.S / 32;
  // iterations 1 .. U-1 run for every wave with no mask: causal, block j + 1
  // lies below the first wave's diagonal block q0 / 32
  const int U = a.causal ? q0 / 32 : nb_wg - 1;
  const int NIT = nb_wg + 1;  // iteration nb_wg adds the last block's P V

  // DMA plan (as in attention_causal_body): a tile is 8 moves of 1 KiB
  constexpr int NM = 32 / 4 / NW;
  static_assert(NM >= 1 && NM * NW * 4 == 32, "moves per wave");
  const int kchunk = (lane & 15) ^ kswz(wave * 4 + (lane >> 4));
  const int vchunk = (lane & 15) ^ vswz(wave * 4 + (lane >> 4));
  const int row0 = wave * 4 + (lane >> 4);
  const uint32_t kbase = (uint32_t)(((int64_t)row0 * a.k_ss + kchunk * 8) * 2);
  const uint32_t vbase = (uint32_t)(((int64_t)row0 * a.v_ss + vchunk * 8) * 2);
  const uint32_t kjs = (uint32_t)(NW * 4 * a.k_ss * 2), vjs = (uint32_t)(NW * 4 * a.v_ss * 2);
  const uint32_t k_lds = lds_addr(KR) + wave * 1024, v_lds = lds_addr(VR) + wave * 1024;
  auto load_k = [&](auto sl, int kb) __attribute__((always_inline)) {
    const uint32_t kst = (uint32_t)((int64_t)kb * 32 * a.k_ss * 2);
    const i32x4_t r = kb < nb_wg ? rk : rnone;
#pragma unroll
    for (int j = 0; j < NM; ++j)
      dma16_asm(r, k_lds + (decltype(sl)::value & 3) * TB + j * NW * 1024, kbase + j * kjs + kst);
  };
  auto load_v = [&](auto sl, int kb) __attribute__((always_inline)) {
    const uint32_t vst = (uint32_t)((int64_t)kb * 32 * a.v_ss * 2);
    const i32x4_t r = kb < nb_wg ? rv : rnone;
#pragma unroll
    for (int j = 0; j < NM; ++j)
      dma16_asm(r, v_lds + (decltype(sl)::value & 3) * TB + j * NW * 1024, vbase + j * vjs + vst);
  };
  // moves an iteration leaves outstanding at its end: the last two
  // iterations' K and V tiles
  constexpr int OUT = 4 * NM;
  // wait until at most n of this wave's DMA moves are outstanding (the Q
  // loads were issued before every move, so they are done by then too)
  auto wait_moves = [&](auto ntag) __attribute__((always_inline)) {
    constexpr int n = decltype(ntag)::value;
    static_assert(n < 16, "vmcnt field");
    __builtin_amdgcn_s_waitcnt(0x0F70 | n);
  };

  const int klb = l32 * 256 + ((lhi ^ (l32 & 1)) << 4);
  const int kx = (l32 & 14) << 4;
  auto koff = [&](int kk) __attribute__((always_inline)) { return klb + ((kk << 5) ^ kx); };
  int vlb, vx;
  {
    const int grp = lane >> 4, gi = lane & 15;
    const int c0 = (grp & 1) * 2 + ((gi & 3) >> 1), vsh = (gi >> 2) & 3;
    vlb = (4 * (grp >> 1) + (gi >> 2)) * 256 + (c0 << 4) + (gi & 1) * 8;
    vx = vsh << 6;
  }
  auto voff = [&](int dt) __attribute__((always_inline)) { return vlb + ((dt << 6) ^ vx); };

  // scores of one block: S^T = K Q^T
  auto qk = [&](const uint8_t *Kt, f32x16 &s) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
    for (int kk = 0; kk < AD / 16; ++kk) {
      const bf16x8_t kf = *reinterpret_cast<const bf16x8_t *>(Kt + koff(kk));
      s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], s, 0, 0, 0);
    }
  };
  // O^T += V^T P^T for one block (P as two 16-key bf16 fragments)
  auto pv = [&](const uint8_t *Vt, const bf16x8_t (&pf)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        s16x4 v[2];
#pragma unroll
        for (int si = 0; si < 2; ++si)
          v[si] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(Vt + (16 * j + 8 * si) * 256 + voff(dt)));
        const bf16x8_t vf = __builtin_shufflevector(__builtin_bit_cast(bf16x4_t, v[0]),
                                                    __builtin_bit_cast(bf16x4_t, v[1]), 0, 1, 2, 3, 4, 5, 6, 7);
        acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[j], acc_o[dt], 0, 0, 0);
      }
  };
  // p = 2^(s c - m) of one block -> bf16 fragments; returns this lane's sum
  auto expblock = [&](const f32x16 &s, bf16x8_t (&pf)[2]) __attribute__((always_inline)) {
    float ps0 = 0.f, ps1 = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * j + e], sl2, -m_run));
        if (e & 1) ps1 += p; else ps0 += p;
        pf[j][e] = (__bf16)p;
      }
    return ps0 + ps1;
  };
  // the softmax of one block (scores s, key block kb); with MASK, keys past
  // klim (the query itself when causal, else the last key) get p = 0
  const int klim = a.causal ? qrow : a.S - 1;
  auto softmax = [&](f32x16 &s, bf16x8_t (&pf)[2], int kb, auto masktag) __attribute__((always_inline)) {
    if constexpr (XF) cast_block(a, s);
    if constexpr (decltype(masktag)::value) {
      // element r holds key kb * 32 + 4 lhi + (8 (r / 4) + r % 4)
      const int t = klim - kb * 32 - lhi * 4;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = ((r >> 2) * 8 + (r & 3)) > t ? -INFINITY : s[r];
    }
    if constexpr (SMX) {
      // e = bf16(exp(bf16(s - m))) in pairs (one packed conversion per
      // rounding); masked keys: s = -inf, d = -inf, e = 0.  The exponential
      // is 2^(d RN(log2 e)), within a few ulp of e^d: the bf16 rounding of
      // e moves only for e^d within those few ulp of a rounding boundary.
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        float d0 = s[r] - mx, d1 = s[r + 1] - mx;
        round_bf16x2(d0, d1);
        float e0 = __builtin_amdgcn_exp2f(d0 * 1.44269504088896340736f);
        float e1 = __builtin_amdgcn_exp2f(d1 * 1.44269504088896340736f);
        round_bf16x2(e0, e1);
        pf[r >> 3][r & 7] = (__bf16)(e0 * rlb);
        pf[r >> 3][(r & 7) + 1] = (__bf16)(e1 * rlb);
      }
      return;
    }
    float ls = expblock(s, pf);
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(!(ls <= 65536.f)) != 0, 0)) {
      // raise m to the block max of the lane pair holding this query, rescale
      // what has been accumulated, recompute the block
      float bm = s[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) bm = fmaxf(bm, s[r]);
      bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
      const float m_new = fmaxf(m_run, bm * sl2);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[t][r] *= alpha;
      l_run *= alpha;
      ls = expblock(s, pf);
    }
    l_run += ls;
  };

  f32x16 sA, sB;
  bf16x8_t pA[2], pB[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pA[j][e] = (__bf16)0.f;
      pB[j][e] = (__bf16)0.f;
    }

  // Iteration j (SL = j mod 4).  Register sets alternate with the parity of
  // j: s_cur holds block j's scores, s_nxt receives block j + 1's; p_cur
  // receives block j's P, p_prev holds block j - 1's.
  auto iter = [&](auto sl, auto gen, int j, f32x16 &s_cur, f32x16 &s_nxt, bf16x8_t (&p_prev)[2],
                  bf16x8_t (&p_cur)[2]) __attribute__((always_inline)) {
    constexpr int SL = decltype(sl)::value;
    constexpr bool GEN = decltype(gen)::value;
    const uint8_t *kn = kslot(SlotTag<SL + 1>{});
    const uint8_t *vp_ = vslot(SlotTag<SL + 3>{});
    if constexpr (!GEN) {
      pv(vp_, p_prev);
      qk(kn, s_nxt);
      softmax(s_cur, p_cur, j, Flag<false>{});
      // order within the block: every LDS fragment read first, a few VALU
      // ops while they land, then each MFMA followed by VALU work (other
      // orders measured within 1%)
      __builtin_amdgcn_sched_group_barrier(0x100, 24, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
      }
    } else if (j <= nb_w) {
      // the same body with the mask; blocks past this wave's last come out
      // as p = 0 (their scores are discarded); no scores past the
      // workgroup's last block, no P V before block 0
      if (j + 1 < nb_wg) qk(kn, s_nxt);
      if (j > 0) pv(vp_, p_prev);
      softmax(s_cur, p_cur, j, Flag<true>{});
    }
    // after the block's MFMAs: a vector memory instruction that waits at
    // issue then holds up no MFMA of this wave; the last iteration moves
    // nothing
    if (j < nb_wg) {
      load_k(SlotTag<SL>{}, j + 4);
      load_v(SlotTag<SL + 2>{}, j + 2);
    }
    wait_moves(SlotTag<OUT>{});
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // prologue: K of blocks 0..3 and V of blocks 0, 1 (in the order that lets
  // each iteration's wait leave exactly the last two iterations' moves
  // outstanding), then the scores of block 0
  load_k(SlotTag<0>{}, 0);
  load_k(SlotTag<1>{}, 1);
  load_k(SlotTag<2>{}, 2);
  load_v(SlotTag<0>{}, 0);
  load_k(SlotTag<3>{}, 3);
  load_v(SlotTag<1>{}, 1);
  wait_moves(SlotTag<OUT>{});
  __builtin_amdgcn_s_barrier();
  qk(kslot(SlotTag<0>{}), sA);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): K0 reads done before its slot is refilled
  __builtin_amdgcn_s_barrier();
  iter(SlotTag<0>{}, Flag<true>{}, 0, sA, sB, pB, pA);
  int j = 1;
  for (; j + 4 <= U; j += 4) {
    iter(SlotTag<1>{}, Flag<false>{}, j, sB, sA, pA, pB);
    iter(SlotTag<2>{}, Flag<false>{}, j + 1, sA, sB, pB, pA);
    iter(SlotTag<3>{}, Flag<false>{}, j + 2, sB, sA, pA, pB);
    iter(SlotTag<0>{}, Flag<false>{}, j + 3, sA, sB, pB, pA);
  }
  // the rest, straight-line (j = 1 mod 4 here): fewer than four uniform
  // iterations, the diagonal blocks and the last P V, at most NW + 4 in all,
  // with the masked body
  static_assert(NW == 4 || NW == 8, "tail length");
  if (j < NIT) iter(SlotTag<1>{}, Flag<true>{}, j, sB, sA, pA, pB);
  if (j + 1 < NIT) iter(SlotTag<2>{}, Flag<true>{}, j + 1, sA, sB, pB, pA);
  if (j + 2 < NIT) iter(SlotTag<3>{}, Flag<true>{}, j + 2, sB, sA, pA, pB);
  if (j + 3 < NIT) iter(SlotTag<0>{}, Flag<true>{}, j + 3, sA, sB, pB, pA);
  if (j + 4 < NIT) iter(SlotTag<1>{}, Flag<true>{}, j + 4, sB, sA, pA, pB);
  if (j + 5 < NIT) iter(SlotTag<2>{}, Flag<true>{}, j + 5, sA, sB, pB, pA);
  if (j + 6 < NIT) iter(SlotTag<3>{}, Flag<true>{}, j + 6, sB, sA, pA, pB);
  if (j + 7 < NIT) iter(SlotTag<0>{}, Flag<true>{}, j + 7, sA, sB, pB, pA);
  if constexpr (NW == 8) {
    if (j + 8 < NIT) iter(SlotTag<1>{}, Flag<true>{}, j + 8, sB, sA, pA, pB);
    if (j + 9 < NIT) iter(SlotTag<2>{}, Flag<true>{}, j + 9, sA, sB, pB, pA);
    if (j + 10 < NIT) iter(SlotTag<3>{}, Flag<true>{}, j + 10, sB, sA, pA, pB);
    if (j + 11 < NIT) iter(SlotTag<0>{}, Flag<true>{}, j + 11, sA, sB, pB, pA);
  }
  wait_moves(SlotTag<0>{});  // no LDS DMA outlives the workgroup

  // normalise (the weights of the bf16 softmax are normalised already) and
  // store
  const float inv_l = SMX ? 1.0f : 1.0f / (l_run + __shfl_xor(l_run, 32, 64));
  uint16_t *orow = op + (int64_t)qrow * a.o_ss;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const uint32_t w0 = pack_bf16x2(acc_o[t][gq * 4 + 0] * inv_l, acc_o[t][gq * 4 + 1] * inv_l);
      const uint32_t w1 = pack_bf16x2(acc_o[t][gq * 4 + 2] * inv_l, acc_o[t][gq * 4 + 3] * inv_l);
      *reinterpret_cast<uint2 *>(orow + t * 32 + gq * 8 + lhi * 4) = make_uint2(w0, w1);
    }
}

// (launch bounds: threads per workgroup, minimum waves per SIMD)
extern "C" __global__ __launch_bounds__(256, 2) void nk_attention_causal_d128_sp(AttnArgs a) {
  attention_sp_body<4>(a);
}
extern "C" __global__ __launch_bounds__(256, 2) void nk_attention_causal_d128_sp_xf(AttnArgs a) {
  attention_sp_body<4, true>(a);
}
extern "C" __global__ __launch_bounds__(256, 2) void nk_attention_causal_d128_sp_xf_bf16(AttnArgs a) {
  attention_sp_body<4, true, true>(a);
}

// ---------------------------------------------------------------------------
// Row statistics of the bf16 softmax (ATT_SOFTMAX_BF16).  Its weights need
// each query's max score, then the sum of its weights, before any weight
// can be formed: two passes over the scores before the weighted values.
// They compute scores only: no V.  Each wave keeps its 32 queries' Q
// fragments in registers; each 32-key K tile moves once per workgroup,
// straight into a four-slot LDS ring (the K layout and moves of the ring
// kernel) three tiles ahead of the one the four waves read.  The keys
// of a query block are cut into chunks of a.ckb blocks, one workgroup per
// (query block, chunk, query head): the longest causal query blocks no
// longer set the length of the launch.  For each chunk and query,
//   MAX  writes the max score: the cast points (bf16 rounding, a positive
//        scale, a correctly rounded divide by a positive divisor) never
//        decrease a score, so the max of the cast scores is the cast of the
//        max of the raw ones, and the cast is applied once;
//   SUM  writes the fp32 sum over the chunk of e = bf16(exp(bf16(s - m))),
//        m the max over the query's chunks.
// Layout of the statistics: AttnArgs::rowstat.  Work items of one (batch,
// KV head) run longest query block first; items are spread over the XCDs
// in contiguous ranges, as in the ring kernel.
// ---------------------------------------------------------------------------
template <bool SUM>
__device__ __forceinline__ void attention_rowstat_body(const AttnArgs &a) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31, lhi = lane >> 5;
  const int nqb = a.S / 128, rep = a.Hq / a.Hkv;

  int per_bg = 0;  // work items of one (batch, KV head)
  for (int qb = 0; qb < nqb; ++qb) per_bg += stat_chunks(a, qb);
  per_bg *= rep;
  const int nwg = a.B * a.Hkv * per_bg;
  int w = blockIdx.x;
  if ((nwg & 7) == 0) w = (w & 7) * (nwg >> 3) + (w >> 3);
  const int bg = w / per_bg;
  if (bg >= a.B * a.Hkv) return;  // (the grid holds exactly nwg workgroups)
  int idx = w % per_bg, qb = nqb - 1;
  for (; qb > 0; --qb) {
    const int n = stat_chunks(a, qb) * rep;
    if (idx < n) break;
    idx -= n;
  }
  const int c = idx / rep, g = bg % a.Hkv, b = bg / a.Hkv;
  const int h = g * rep + idx % rep;
  if (c >= stat_chunks(a, qb)) return;  // (likewise)

  // this wave's blocks of the chunk: every one of the chunk's, up to the
  // block holding its own queries (causal); never empty, as a causal
  // chunk starts at or before the query block's first key block
  const int wq0 = qb * 128 + wave * 32, qrow = wq0 + l32;
  const int kb0 = c * a.ckb;
  int kb1 = min(kb0 + a.ckb, a.causal ? (qb + 1) * 4 : a.S / 32);
  if (a.causal) kb1 = min(kb1, wq0 / 32 + 1);

  const int kb1_wg = min(kb0 + a.ckb, a.causal ? (qb + 1) * 4 : a.S / 32);  // the workgroup's blocks
  const uint16_t *qp = a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh;
  const uint16_t *kp = a.k + (int64_t)b * a.k_sb + (int64_t)g * a.k_sh;
  const i32x4_t rk = rsrc_words(kp, (int64_t)a.S * a.k_ss * 2);
  const i32x4_t rnone = rsrc_words(kp, 0);  // moves of no bytes: zeros, no memory read
  constexpr int TB = 32 * AD * 2;  // one K tile
  __shared__ __attribute__((aligned(1024))) uint8_t KT[4 * TB];
  const int64_t nq = (int64_t)a.B * a.Hq * a.S;
  float *st = a.rowstat + ((int64_t)b * a.Hq + h) * a.S + qrow;
  bf16x8_t qf[AD / 16];  // loaded once the first moves are out
  float mx = 0.f;        // SUM: the query's max score, likewise

  // tile moves (two 1 KiB moves per wave): move j of wave w fills key rows
  // 16 j + 4 w .. + 3, lane l the row's 16-byte position l % 16, which
  // holds chunk (l % 16) ^ (row % 16): chunk c of row r sits at
  // r * 256 + 16 (c ^ (r % 16))
  const int row0 = wave * 4 + (lane >> 4);
  const int tch = (lane & 15) ^ (row0 & 15);  // (row0 + 16 j has the same low bits)
  const uint32_t tsrc = (uint32_t)(((int64_t)row0 * a.k_ss + tch * 8) * 2);
  const uint32_t tjs = (uint32_t)((int64_t)16 * a.k_ss * 2), tstep = (uint32_t)((int64_t)32 * a.k_ss * 2);
  const uint32_t tlds = lds_addr(KT) + wave * 1024;
  auto move = [&](int t) __attribute__((always_inline)) {  // tile t of the chunk into slot t % 4
    const int kb = kb0 + t;
    const i32x4_t r = t < kb1_wg - kb0 ? rk : rnone;
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16_asm(r, tlds + (t & 3) * TB + j * 4096, tsrc + j * tjs + kb * tstep);
  };
  // this lane's fragment kk of a tile: row l32, chunk 2 kk + lhi
  auto koff = [&](int kk) __attribute__((always_inline)) { return l32 * 256 + 16 * ((2 * kk + lhi) ^ (l32 & 15)); };
  float acc = SUM ? 0.f : -INFINITY;
  auto block = [&](int kb, const uint8_t *Kt) __attribute__((always_inline)) {
    f32x16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
    for (int kk = 0; kk < AD / 16; ++kk)
      s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*reinterpret_cast<const bf16x8_t *>(Kt + koff(kk)), qf[kk], s,
                                                  0, 0, 0);
    if constexpr (SUM) cast_block(a, s);
    if (a.causal && kb == wq0 / 32) {
      // element r holds key kb * 32 + 4 lhi + (8 (r / 4) + r % 4)
      const int t = qrow - kb * 32 - lhi * 4;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = ((r >> 2) * 8 + (r & 3)) > t ? -INFINITY : s[r];
    }
    if constexpr (SUM) {
      float ps0 = 0.f, ps1 = 0.f;
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        float d0 = s[r] - mx, d1 = s[r + 1] - mx;
        round_bf16x2(d0, d1);
        float e0 = __builtin_amdgcn_exp2f(d0 * 1.44269504088896340736f);
        float e1 = __builtin_amdgcn_exp2f(d1 * 1.44269504088896340736f);
        round_bf16x2(e0, e1);
        ps0 += e0;
        ps1 += e1;
      }
      acc += ps0 + ps1;
    } else {
      float bm = s[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) bm = fmaxf(bm, s[r]);
      acc = fmaxf(acc, bm);
    }
  };
  // tile t = kb - kb0 lands in slot t % 4.  Step t moves tile t + 3 into
  // the slot of tile t - 1 (every wave finished it before the last
  // barrier), reads tile t, then waits until tile t + 1 has landed: each
  // step issues two moves per wave (of no bytes past the chunk), so at most
  // the four of tiles t + 2 and t + 3 may still be in flight.
  const int nt = kb1_wg - kb0;
  move(0);
  move(1);
  move(2);
  // Q fragments (and the query's max score), all in hand before the loop:
  // the compiler, which cannot count the moves, then adds no wait of its
  // own inside the loop
#pragma unroll
  for (int kk = 0; kk < AD / 16; ++kk)
    qf[kk] = *reinterpret_cast<const bf16x8_t *>(qp + (int64_t)qrow * a.q_ss + kk * 16 + lhi * 8);
  if constexpr (SUM) {
    const int nc = stat_chunks(a, qb);
    mx = st[0];
    for (int cc = 1; cc < nc; ++cc) mx = fmaxf(mx, st[cc * nq]);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the moves of tiles 0 - 2 as well
#pragma unroll
  for (int kk = 0; kk < AD / 16; ++kk) asm volatile("" ::"v"(qf[kk]));
  asm volatile("" ::"v"(mx));
  __syncthreads();
  for (int t = 0; t < nt; ++t) {
    move(t + 3);
    if (kb0 + t < kb1) block(kb0 + t, KT + (t & 3) * TB);
    __builtin_amdgcn_s_waitcnt(0x0F70 | 4);  // vmcnt(4): tile t + 1 done
    __syncthreads();
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): no move outlives the workgroup
  if constexpr (SUM) {
    acc += __shfl_xor(acc, 32, 64);
    if (lhi == 0) st[(a.nch + c) * nq] = acc;
  } else {
    acc = fmaxf(acc, __shfl_xor(acc, 32, 64));
    if (lhi == 0) st[c * nq] = cast_score(a, acc);
  }
}
extern "C" __global__ __launch_bounds__(256) void nk_attention_rowmax_d128(AttnArgs a) {
  attention_rowstat_body<false>(a);
}
extern "C" __global__ __launch_bounds__(256) void nk_attention_rowsum_d128(AttnArgs a) {
  attention_rowstat_body<true>(a);
}
extern "C" __global__ __launch_bounds__(512, 1) void nk_attention_causal_d128_sp8(AttnArgs a) {
  attention_sp_body<8>(a);
}
extern "C" __global__ __launch_bounds__(256, 2) void nk_attention_causal_d128(AttnArgs a) {
  attention_causal_body<4, 64, true>(a);
}
extern "C" __global__ __launch_bounds__(512, 2) void nk_attention_causal_d128_w8(AttnArgs a) {
  attention_causal_body<8, 64, true>(a);
}
extern "C" __global__ __launch_bounds__(256, 3) void nk_attention_causal_d128_k32(AttnArgs a) {
  attention_causal_body<4, 32, false>(a);
}

// ---------------------------------------------------------------------------
// Decode attention: one query token per sequence against a KV cache,
//   o[b, h] = softmax(q[b, h] . K[b, 0..pos, h / rep]^T * scale) V[b, 0..pos, h / rep]
// with rep = Hq / Hkv query heads per KV head and pos read from device memory
// (the keys after it are the ones the causal mask row of position pos adds
// -1e5 to: they contribute nothing).  The cast points of the traced NumPy
// code are kept by flags: the q.k product rounded to bf16, the scaled score
// rounded to bf16, and softmax with bf16 results per operation (s - m,
// exp, the fp32-accumulated sum, the quotient); the weighted sum of values
// accumulates in fp32.
//
// One token's attention is little work spread over a long cache, so the
// keys are cut into splits of DKS = 128 (the cache length fixes the grid;
// splits past pos exit at once) and the step runs as four launches over a
// workspace (DecodeAttnArgs::ws):
//   scores   one workgroup per (batch, KV head, split): the split's K rows
//            read into registers (16 bytes per lane), fp32 dot products
//            with q from LDS, reduced over the 16 lanes of a row, the cast
//            points; the scores and each query's max over the split go to
//            the workspace;
//   rowstat  one workgroup per (batch, query head): the row's max m over
//            the split maxima and the sum l of e = exp(s - m) (block
//            reduction), each step rounded to bf16 with DEC_SOFTMAX_BF16;
//   values   one workgroup per (batch, KV head, split): the split's V rows
//            read into registers and its weights p = e / l (again each step
//            rounded with DEC_SOFTMAX_BF16) from the scores, m and l into
//            LDS; fp32 sums of p v over key groups added in a fixed order,
//            written per split;
//   combine  one workgroup per (batch, query head): the splits' partial
//            outputs added in split order, rounded to bf16.
// Workspace (fp32), with nsplit = ceil(Smax / DKS) and rows r = b * Hq + h:
//   scores            [r][Smax] at 0
//   split maxima      [r][nsplit] after B * Hq * Smax
//   partial outputs   [r][nsplit][128] after that
//   row statistics    [r][2] (m, l) after that
#define DQ_MAX 16       // query heads per KV head (kernels for 1, 2, 4, 8, 16)
#define DKS 128         // keys per split

enum { DEC_RND_PROD = 1, DEC_RND_SCORE = 2, DEC_SOFTMAX_BF16 = 4, DEC_DIVIDE = 8 };

struct DecodeAttnArgs {
  const uint16_t *q;   // (B, Hq, 128): q_sb, q_sh
  const uint16_t *k;   // cache (B, Smax, Hkv, 128): k_sb, k_ss, k_sh
  const uint16_t *v;   // v_sb, v_ss, v_sh
  uint16_t *o;         // (B, Hq, 128): o_sb, o_sh
  const int32_t *pos;  // last attended position (one value for every sequence)
  int64_t q_sb, q_sh, k_sb, k_ss, k_sh, v_sb, v_ss, v_sh, o_sb, o_sh;
  int32_t B, Smax, Hq, Hkv;
  float scale;  // multiplied in (divided by with DEC_DIVIDE)
  int32_t flags;
  float *ws;    // workspace (see above)
  int32_t nsplit;
};

__device__ __forceinline__ float bf16r(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// attended keys: pos + 1, pos clamped into the cache
__device__ __forceinline__ int decode_keys(const DecodeAttnArgs &a) {
  int pos = *a.pos;
  pos = pos < 0 ? 0 : (pos >= a.Smax ? a.Smax - 1 : pos);
  return pos + 1;
}

// Scores: lane (r, c) of wave w, r = lane / 4, c = lane % 4, holds dims
// 8 (c + 4 j) .. +7 (j < 4) of keys w * 32 + r + 16 i (i < 2), read
// straight from the cache (each load instruction covers 64 contiguous
// bytes of 16 rows); q of the REPT queries comes from LDS.  A key's dot
// product is the quad's four partial sums added by two DPP steps (the four
// lanes then hold the same sum), whose cast points each lane applies; lane
// c = 0 stores.  2 KiB of LDS per workgroup at REPT = 4.
template <int REPT>
__device__ __forceinline__ void decode_scores_body(const DecodeAttnArgs &a) {
  __shared__ __attribute__((aligned(16))) float qs[REPT][AD];
  __shared__ float smax[4][REPT];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rep = a.Hq / a.Hkv;  // <= REPT
  const int sp = blockIdx.x % a.nsplit;
  const int bg = blockIdx.x / a.nsplit;
  const int b = bg / a.Hkv, g = bg % a.Hkv;
  const int L = decode_keys(a);
  const int k0 = sp * DKS;
  if (k0 >= L) return;  // uniform: the whole workgroup
  const int nk = min(DKS, L - k0);
  const uint16_t *kb = a.k + (int64_t)b * a.k_sb + (int64_t)g * a.k_sh + (int64_t)k0 * a.k_ss;
  const int r = lane >> 2, c = lane & 3;

  // every load before the first use: K (rows past pos load the last
  // attended row, their scores are dropped), then q (thread -> 8 values of
  // one query)
  uint4 kr[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = min(wave * 32 + r + 16 * i, nk - 1);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      kr[i][j] = *reinterpret_cast<const uint4 *>(kb + (int64_t)row * a.k_ss + (c + 4 * j) * 8);
  }
  {
    const int qi = tid >> 4, qc = tid & 15;
    if (qi < REPT) {
      const int qq = min(qi, rep - 1);
      const uint4 qw = *reinterpret_cast<const uint4 *>(a.q + (int64_t)b * a.q_sb +
                                                        (int64_t)(g * rep + qq) * a.q_sh + qc * 8);
      float *qd = &qs[qi][qc * 8];
      qd[0] = __uint_as_float(qw.x << 16); qd[1] = __uint_as_float(qw.x & 0xffff0000u);
      qd[2] = __uint_as_float(qw.y << 16); qd[3] = __uint_as_float(qw.y & 0xffff0000u);
      qd[4] = __uint_as_float(qw.z << 16); qd[5] = __uint_as_float(qw.z & 0xffff0000u);
      qd[6] = __uint_as_float(qw.w << 16); qd[7] = __uint_as_float(qw.w & 0xffff0000u);
    }
  }
  __syncthreads();

  float kf[2][4][8];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 w = kr[i][j];
      kf[i][j][0] = __uint_as_float(w.x << 16); kf[i][j][1] = __uint_as_float(w.x & 0xffff0000u);
      kf[i][j][2] = __uint_as_float(w.y << 16); kf[i][j][3] = __uint_as_float(w.y & 0xffff0000u);
      kf[i][j][4] = __uint_as_float(w.z << 16); kf[i][j][5] = __uint_as_float(w.z & 0xffff0000u);
      kf[i][j][6] = __uint_as_float(w.w << 16); kf[i][j][7] = __uint_as_float(w.w & 0xffff0000u);
    }
  const int64_t row0 = (int64_t)b * a.Hq + g * rep;  // score row of query 0
  float *sc = a.ws + row0 * a.Smax + k0;
  float mloc[REPT];
#pragma unroll
  for (int q = 0; q < REPT; ++q) {
    float qv[4][8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 lo = *reinterpret_cast<const float4 *>(&qs[q][(c + 4 * j) * 8]);
      const float4 hi = *reinterpret_cast<const float4 *>(&qs[q][(c + 4 * j) * 8 + 4]);
      qv[j][0] = lo.x; qv[j][1] = lo.y; qv[j][2] = lo.z; qv[j][3] = lo.w;
      qv[j][4] = hi.x; qv[j][5] = hi.y; qv[j][6] = hi.z; qv[j][7] = hi.w;
    }
    mloc[q] = -INFINITY;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = wave * 32 + r + 16 * i;
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(qv[j][e], kf[i][j][e], d);
      d = d + dpp<0xB1>(d);  // the quad's sum: the same value in its four lanes
      d = d + dpp<0x4E>(d);
      float s = d;
      if (a.flags & DEC_RND_PROD) s = bf16r(s);
      s = (a.flags & DEC_DIVIDE) ? s / a.scale : s * a.scale;
      if (a.flags & DEC_RND_SCORE) s = bf16r(s);
      if (c == 0 && q < rep && key < nk) sc[(int64_t)q * a.Smax + key] = s;
      if (key < nk) mloc[q] = fmaxf(mloc[q], s);
    }
  }
  // the split's max per query: over the 16 key rows of the wave, then over
  // the waves
#pragma unroll
  for (int q = 0; q < REPT; ++q) {
    float m = mloc[q];
#pragma unroll
    for (int off = 4; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (lane == 0) smax[wave][q] = m;
  }
  __syncthreads();
  if (tid < rep) {
    float *mx = a.ws + (int64_t)a.B * a.Hq * a.Smax + row0 * a.nsplit + sp;
    mx[(int64_t)tid * a.nsplit] = fmaxf(fmaxf(smax[0][tid], smax[1][tid]), fmaxf(smax[2][tid], smax[3][tid]));
  }
}

extern "C" __global__ __launch_bounds__(256) void nk_decode_rowstat_d128(DecodeAttnArgs a) {
  __shared__ float red[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;  // b * Hq + h
  const int L = decode_keys(a);
  const int nsp = (L + DKS - 1) / DKS;
  const bool rnd = (a.flags & DEC_SOFTMAX_BF16) != 0;
  const float *sc = a.ws + row * a.Smax;
  const float *mx = a.ws + (int64_t)a.B * a.Hq * a.Smax + row * a.nsplit;
  constexpr int U = 16;  // loads of a batch first: one latency for 4096 keys
  // the first batch of scores is loaded with the split maxima (it does not
  // depend on the max); the maxima are shared out over the threads, then
  // the workgroup's max
  float x[U];
#pragma unroll
  for (int u = 0; u < U; ++u) x[u] = sc[min(u * 256 + tid, L - 1)];
  __shared__ float mred[4];
  float m = -INFINITY;
  for (int i = tid; i < nsp; i += 256) m = fmaxf(m, mx[i]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if (lane == 0) mred[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(mred[0], mred[1]), fmaxf(mred[2], mred[3]));
  float sum = 0.f;
  for (int j0 = 0; j0 < L; j0 += 256 * U) {
    if (j0 > 0) {
#pragma unroll
      for (int u = 0; u < U; ++u) x[u] = sc[min(j0 + u * 256 + tid, L - 1)];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (j0 + u * 256 + tid < L) {
        float d = x[u] - m;
        if (rnd) d = bf16r(d);
        float e = expf(d);
        if (rnd) e = bf16r(e);
        sum += e;
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  if (tid == 0) {
    sum = (red[0] + red[1]) + (red[2] + red[3]);
    if (rnd) sum = bf16r(sum);
    float *rs = a.ws + (int64_t)a.B * a.Hq * (a.Smax + a.nsplit + (int64_t)a.nsplit * AD) + row * 2;
    rs[0] = m;
    rs[1] = sum;
  }
}

// Weighted values: the split's weights p (REPT per key, 0 past pos or rep)
// into LDS first; lane (c, r) of wave w holds columns 8c .. 8c+7 of keys
// w * 32 + r + 4 i (i < 8), read straight from the cache with the scores
// and statistics (every load issued before the first use), and sums p v
// over its keys in order; the four key groups of a wave are added by xor
// shuffles (16, then 32), the four waves through LDS as (w0 + w1) +
// (w2 + w3).  10 KiB of LDS per workgroup at REPT = 4.
template <int REPT>
__device__ __forceinline__ void decode_values_body(const DecodeAttnArgs &a) {
  __shared__ __attribute__((aligned(16))) float ps[DKS][REPT];
  __shared__ float red[4][REPT][AD];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rep = a.Hq / a.Hkv;  // <= REPT
  const int sp = blockIdx.x % a.nsplit;
  const int bg = blockIdx.x / a.nsplit;
  const int b = bg / a.Hkv, g = bg % a.Hkv;
  const int L = decode_keys(a);
  const int k0 = sp * DKS;
  if (k0 >= L) return;
  const int nk = min(DKS, L - k0);
  const uint16_t *vb = a.v + (int64_t)b * a.v_sb + (int64_t)g * a.v_sh + (int64_t)k0 * a.v_ss;
  const int64_t row0 = (int64_t)b * a.Hq + g * rep;
  const float *pw = a.ws + row0 * a.Smax + k0;
  const int c = lane & 15, r = lane >> 4;

  uint4 vr[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = min(wave * 32 + r + 4 * i, nk - 1);
    vr[i] = *reinterpret_cast<const uint4 *>(vb + (int64_t)row * a.v_ss + c * 8);
  }
  {
    // this thread's (key kk, queries q0, q0 + 2, ...) weights
    constexpr int NJ = (REPT + 1) / 2;
    const int kk = tid & (DKS - 1), q0 = tid >> 7;
    const float *rs = a.ws + (int64_t)a.B * a.Hq * (a.Smax + a.nsplit + (int64_t)a.nsplit * AD) + row0 * 2;
    float pv[NJ], st[NJ][2];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int qc = min(q0 + 2 * j, rep - 1);
      pv[j] = pw[(int64_t)qc * a.Smax + min(kk, nk - 1)];
      st[j][0] = rs[qc * 2];
      st[j][1] = rs[qc * 2 + 1];
    }
    const bool rnd = (a.flags & DEC_SOFTMAX_BF16) != 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int qi = q0 + 2 * j;
      if (qi < REPT) {
        float p = 0.f;  // (keys past pos, queries past rep: weight 0)
        if (kk < nk && qi < rep) {
          float d = pv[j] - st[j][0];
          if (rnd) d = bf16r(d);
          float e = expf(d);
          if (rnd) e = bf16r(e);
          p = e / st[j][1];
          if (rnd) p = bf16r(p);
        }
        ps[kk][qi] = p;
      }
    }
  }
  __syncthreads();

  float acc[REPT][8];
#pragma unroll
  for (int q = 0; q < REPT; ++q)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[q][e] = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int key = wave * 32 + r + 4 * i;
    const bool in = key < nk;  // rows past pos: weight 0 and values 0
    float vv[8];
    vv[0] = __uint_as_float(vr[i].x << 16); vv[1] = __uint_as_float(vr[i].x & 0xffff0000u);
    vv[2] = __uint_as_float(vr[i].y << 16); vv[3] = __uint_as_float(vr[i].y & 0xffff0000u);
    vv[4] = __uint_as_float(vr[i].z << 16); vv[5] = __uint_as_float(vr[i].z & 0xffff0000u);
    vv[6] = __uint_as_float(vr[i].w << 16); vv[7] = __uint_as_float(vr[i].w & 0xffff0000u);
#pragma unroll
    for (int e = 0; e < 8; ++e) vv[e] = in ? vv[e] : 0.f;
#pragma unroll
    for (int q = 0; q < REPT; ++q) {
      const float p = ps[key][q];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[q][e] = fmaf(p, vv[e], acc[q][e]);
    }
  }
#pragma unroll
  for (int q = 0; q < REPT; ++q)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[q][e];
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      acc[q][e] = v;
    }
  if (r == 0) {
#pragma unroll
    for (int q = 0; q < REPT; ++q)
#pragma unroll
      for (int e = 0; e < 8; ++e) red[wave][q][c * 8 + e] = acc[q][e];
  }
  __syncthreads();
  const int d = tid & (AD - 1), qh = tid >> 7;
  float *op = a.ws + (int64_t)a.B * a.Hq * (a.Smax + a.nsplit) + (row0 * a.nsplit + sp) * AD;
  for (int q = qh; q < rep; q += 2)
    op[(int64_t)q * a.nsplit * AD + d] = (red[0][q][d] + red[1][q][d]) + (red[2][q][d] + red[3][q][d]);
}

// kernels for up to REPT query heads per KV head
#define NK_DECODE_REP(R)                                                                           \
  extern "C" __global__ __launch_bounds__(256) void nk_decode_scores_d128_r##R(DecodeAttnArgs a) { \
    decode_scores_body<R>(a);                                                                      \
  }                                                                                                \
  extern "C" __global__ __launch_bounds__(256) void nk_decode_values_d128_r##R(DecodeAttnArgs a) { \
    decode_values_body<R>(a);                                                                      \
  }
NK_DECODE_REP(1)
NK_DECODE_REP(2)
NK_DECODE_REP(4)
NK_DECODE_REP(8)
NK_DECODE_REP(16)

extern "C" __global__ __launch_bounds__(128) void nk_decode_combine_d128(DecodeAttnArgs a) {
  const int d = threadIdx.x;
  const int64_t row = blockIdx.x;  // b * Hq + h
  const int b = (int)(row / a.Hq), h = (int)(row % a.Hq);
  const int nsp = (decode_keys(a) + DKS - 1) / DKS;
  const float *op = a.ws + (int64_t)a.B * a.Hq * (a.Smax + a.nsplit) + row * a.nsplit * AD + d;
  float o = 0.f;
  for (int i0 = 0; i0 < nsp; i0 += 32) {  // loads of a batch first (32 splits: 4096 keys), added in split order
    float x[32];
#pragma unroll
    for (int u = 0; u < 32; ++u) x[u] = op[(int64_t)min(i0 + u, nsp - 1) * AD];
#pragma unroll
    for (int u = 0; u < 32; ++u)
      if (i0 + u < nsp) o += x[u];
  }
  a.o[(int64_t)b * a.o_sb + (int64_t)h * a.o_sh + d] = f32_to_bf16(o);
}
