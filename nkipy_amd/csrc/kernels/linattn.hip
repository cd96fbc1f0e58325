// Chunked causal linear attention for gfx950.
//
//   phi(x) = elu(x) + 1 = (x > 0 ? x + 1 : exp(x))
//   o_t = phi(q_t)^T S_t / (phi(q_t)^T z_t),
//   S_t = sum_{s <= t} phi(k_s) v_s^T  (d x d_v, fp32),  z_t = sum_{s <= t} phi(k_s)
//
// Chunked form (chunk C = 64): for chunk c with rows t of the chunk,
//   O_c = phi(Q_c) S_{c-1} + tril(phi(Q_c) phi(K_c)^T) V_c
//   den = phi(Q_c) z_{c-1} + rowsum(tril(phi(Q_c) phi(K_c)^T))
//   S_c = S_{c-1} + phi(K_c)^T V_c,   z_c = z_{c-1} + colsum(phi(K_c))
// (no reference kernel computes this; the nearest analogue is the recurrent
// DeltaNet kernel, examples/linear_attention/deltanet.py:74-128).
//
// Layout: q, k, v, o are (B*H, T, 128) row-major bf16.  One workgroup of 4
// waves owns one (b, h) sequence and a 32-column slice of d_v, so the four
// slices of a head run as four workgroups (256 workgroups for B*H = 64) and
// each keeps its 128 x 32 fp32 state slice in MFMA accumulator registers for
// the whole sequence.  Per chunk: the next chunk's q / k / v tile is fetched
// into registers while the current one is processed; phi is applied on the
// way into LDS; A = phi(Q) phi(K)^T (32x32x16 MFMA), phi(Q) S (16x16x32),
// A V (16x16x32) and the state update phi(K)^T V (32x32x16) run on fp16 MFMA
// with fp32 accumulation; the normaliser is a VALU dot product; the output
// tile is staged in LDS and written with 16-byte stores.  The state enters
// the phi(Q) S product as an fp16 copy (double-buffered in LDS); the running
// state itself stays fp32.
//
// MFMA operands are fp16, not bf16: phi(x) = 1 + x + ... for the small inputs
// of attention, so the information sits in deviations from 1 and in
// A = phi(Q) phi(K)^T ~ d + small terms; bf16's 8-bit significand loses about
// 5% of those deviations, fp16's 11 bits keep the output within 0.4% of the
// fp32 recurrence (same MFMA rate on gfx950).  Limit: the fp16 state copy
// overflows if an entry of S exceeds 65504.

#include "common.h"

using namespace nk;

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define LC 64    // chunk length
#define LD 128   // head dim (q, k)
#define LDV 128  // head dim (v, o)
#define LS 32    // d_v columns per workgroup

struct LinAttnArgs {
  const uint16_t *q;
  const uint16_t *k;
  const uint16_t *v;
  uint16_t *o;
  int64_t BH;      // batch * heads
  int64_t T;       // sequence length (multiple of 64)
};

// swizzled element offsets of the LDS tiles (16-byte chunks permuted by row)
__device__ __forceinline__ int off128(int row, int col) {  // rows of 128 16-bit values
  return row * 128 + ((((col >> 3) ^ (row & 15))) << 3) + (col & 7);
}
__device__ __forceinline__ int off64(int row, int col) {  // rows of 64 16-bit values
  return row * 64 + ((((col >> 3) ^ ((row >> 1) & 7))) << 3) + (col & 7);
}

__device__ __forceinline__ float phi(float x) { return x > 0.f ? x + 1.f : __expf(x); }

extern "C" __global__ __launch_bounds__(256, 1) void nk_linattn_c64_d128(LinAttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t Qs[LC * LD];       // [t][d]
  __shared__ __attribute__((aligned(16))) uint16_t Ks[LC * LD];       // [s][d]
  __shared__ __attribute__((aligned(16))) uint16_t Kts[LD * LC];      // [d][s]
  __shared__ __attribute__((aligned(16))) uint16_t Vts[LS * LC];      // [j][s]
  __shared__ __attribute__((aligned(16))) uint16_t As[LC * LC];       // [t][s]
  __shared__ __attribute__((aligned(16))) uint16_t St[2][LS * LD];    // [j][d]
  __shared__ __attribute__((aligned(16))) uint16_t Os[LC * LS];       // [t][j]
  __shared__ float zs[2][LD];
  __shared__ float dens[LC];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, lhi = lane >> 5;
  const int l16 = lane & 15, lq = lane >> 4;
  // The four d_v slices of a head read the same q / k tiles: give them
  // workgroup ids that are equal modulo 8 so they land on the same XCD and
  // share its L2 (workgroups are dealt to the 8 XCDs round robin).
  int64_t bh;
  int slice;
  if ((a.BH & 7) == 0) {
    const int id = blockIdx.x;
    bh = (int64_t)(id >> 5) * 8 + (id & 7);
    slice = (id >> 3) & 3;
  } else {
    bh = blockIdx.x >> 2;
    slice = blockIdx.x & 3;
  }
  const int j0 = slice * LS;
  const int64_t base = bh * a.T * LD;
  const int nchunks = (int)(a.T / LC);

  // state accumulator: rows d = wave*32 + ..., cols j (32), fp32
  f32x16 S;
#pragma unroll
  for (int r = 0; r < 16; ++r) S[r] = 0.f;
  if (tid < LD) zs[0][tid] = 0.f;
  for (int i = tid; i < LS * LD; i += 256) St[0][i] = 0;  // S_0 = 0 (fp16 zero bits)

  // register staging: two chunks in flight (prefetch distance 2)
  uint4 rqA[4], rkA[4], rvA, rqB[4], rkB[4], rvB;
  auto load_chunk = [&](int c, uint4 (&rq)[4], uint4 (&rk)[4], uint4 &rv) {
    const int64_t cb = base + (int64_t)c * LC * LD;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ci = tid + 256 * i;
      const int row = ci >> 4, col = (ci & 15) * 8;
      rq[i] = *reinterpret_cast<const uint4 *>(a.q + cb + row * LD + col);
      rk[i] = *reinterpret_cast<const uint4 *>(a.k + cb + row * LD + col);
    }
    const int vrow = tid >> 2, vcol = j0 + (tid & 3) * 8;
    rv = *reinterpret_cast<const uint4 *>(a.v + cb + vrow * LDV + vcol);
  };

  auto body = [&](int c, uint4 (&rq)[4], uint4 (&rk)[4], uint4 &rv) {
    const int cur = c & 1, nxt = cur ^ 1;
    // ---- step 1: phi and staging into LDS ---------------------------------
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ci = tid + 256 * i;
      const int row = ci >> 4, col = (ci & 15) * 8;
      float fq[8], fk[8];
      Raw8<bf16> rr;
      rr.w[0] = rq[i];
      decode8(rr, fq);
      rr.w[0] = rk[i];
      decode8(rr, fk);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        fq[e] = phi(fq[e]);
        fk[e] = phi(fk[e]);
      }
      Raw8<f16> oq, ok;
      encode8(fq, oq);
      encode8(fk, ok);
      *reinterpret_cast<uint4 *>(Qs + off128(row, col)) = oq.w[0];
      *reinterpret_cast<uint4 *>(Ks + off128(row, col)) = ok.w[0];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        Kts[off64(col + e, row)] = (uint16_t)h16_of(ok.w[0], e);
    }
    {
      const int vrow = tid >> 2, vc = (tid & 3) * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        Vts[off64(vc + e, vrow)] = f32_to_f16(bf16_to_f32((uint16_t)h16_of(rv, e)));
    }
    if (c + 2 < nchunks) load_chunk(c + 2, rq, rk, rv);
    __syncthreads();  // B1
    // flush the previous chunk's output tile (staged in Os)
    if (c > 0) {
      const int row = tid >> 2, part = (tid & 3) * 8;
      const int64_t o_off = base + ((int64_t)(c - 1) * LC + row) * LDV + j0 + part;
      nt_store16(a.o + o_off, *reinterpret_cast<const uint4 *>(Os + row * LS + part));
    }

    // ---- step 2a: A = phi(Q) phi(K)^T (wave tile (wave>>1, wave&1)), masked
    {
      const int ti = wave >> 1, tj = wave & 1;
      f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
      for (int kk = 0; kk < LD / 16; ++kk) {
        const int col = kk * 16 + lhi * 8;
        f16x8_t af = *reinterpret_cast<const f16x8_t *>(Qs + off128(ti * 32 + l32, col));
        f16x8_t bf = *reinterpret_cast<const f16x8_t *>(Ks + off128(tj * 32 + l32, col));
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc, 0, 0, 0);
      }
      const int s = tj * 32 + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = ti * 32 + (r >> 2) * 8 + lhi * 4 + (r & 3);
        const float val = (s <= t) ? acc[r] : 0.f;
        As[off64(t, s)] = f32_to_f16(val);
      }
    }
    // ---- step 2b: O = phi(Q) S_prev (rows wave*16.., both 16-col tiles) ----
    f32x4 o0, o1;
#pragma unroll
    for (int r = 0; r < 4; ++r) { o0[r] = 0.f; o1[r] = 0.f; }
    {
      const uint16_t *st = St[cur];
#pragma unroll
      for (int kk = 0; kk < LD / 32; ++kk) {
        const int col = kk * 32 + lq * 8;
        f16x8_t af = *reinterpret_cast<const f16x8_t *>(Qs + off128(wave * 16 + l16, col));
        f16x8_t b0 = *reinterpret_cast<const f16x8_t *>(st + off128(l16, col));
        f16x8_t b1 = *reinterpret_cast<const f16x8_t *>(st + off128(16 + l16, col));
        o0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, b0, o0, 0, 0, 0);
        o1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, b1, o1, 0, 0, 0);
      }
    }
    // ---- step 2c: state update S += phi(K)^T V; fp16 copy for the next chunk
    {
#pragma unroll
      for (int kk = 0; kk < LC / 16; ++kk) {
        const int col = kk * 16 + lhi * 8;
        f16x8_t af = *reinterpret_cast<const f16x8_t *>(Kts + off64(wave * 32 + l32, col));
        f16x8_t bf = *reinterpret_cast<const f16x8_t *>(Vts + off64(l32, col));
        S = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, S, 0, 0, 0);
      }
      uint16_t *stn = St[nxt];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = wave * 32 + (r >> 2) * 8 + lhi * 4 + (r & 3);
        stn[off128(l32, d)] = f32_to_f16(S[r]);
      }
    }
    // ---- step 2d: z_next = z + colsum(phi(K)) (fp16 values, as in S) -------
    if (tid < LD) {
      float zsum = zs[cur][tid];
#pragma unroll
      for (int s8 = 0; s8 < LC / 8; ++s8) {
        float f[8];
        Raw8<f16> rr;
        rr.w[0] = *reinterpret_cast<const uint4 *>(Kts + off64(tid, s8 * 8));
        decode8(rr, f);
#pragma unroll
        for (int e = 0; e < 8; ++e) zsum += f[e];
      }
      zs[nxt][tid] = zsum;
    }
    __syncthreads();  // B2: As complete

    // ---- step 3a: O += A V ------------------------------------------------
#pragma unroll
    for (int kk = 0; kk < LC / 32; ++kk) {
      const int col = kk * 32 + lq * 8;
      f16x8_t af = *reinterpret_cast<const f16x8_t *>(As + off64(wave * 16 + l16, col));
      f16x8_t b0 = *reinterpret_cast<const f16x8_t *>(Vts + off64(l16, col));
      f16x8_t b1 = *reinterpret_cast<const f16x8_t *>(Vts + off64(16 + l16, col));
      o0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, b0, o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, b1, o1, 0, 0, 0);
    }
    // ---- step 3b: den[t] = phi(q_t) . z_prev + rowsum(A[t]) ---------------
    {
      const int t = tid >> 2, p = tid & 3;
      float acc = 0.f;
      // intra: 16 columns of A
#pragma unroll
      for (int s8 = 0; s8 < 2; ++s8) {
        float f[8];
        Raw8<f16> rr;
        rr.w[0] = *reinterpret_cast<const uint4 *>(As + off64(t, p * 16 + s8 * 8));
        decode8(rr, f);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += f[e];
      }
      // inter: 32 feature dims
      const float *z = zs[cur];
#pragma unroll
      for (int d8 = 0; d8 < 4; ++d8) {
        float f[8];
        Raw8<f16> rr;
        const int d0 = p * 32 + d8 * 8;
        rr.w[0] = *reinterpret_cast<const uint4 *>(Qs + off128(t, d0));
        decode8(rr, f);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fmaf(f[e], z[d0 + e], acc);
      }
      acc += __shfl_xor(acc, 1, 64);
      acc += __shfl_xor(acc, 2, 64);
      if (p == 0) dens[t] = acc;
    }
    __syncthreads();  // B3: dens complete

    // ---- step 4: normalise and stage the output tile ----------------------
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = wave * 16 + lq * 4 + r;
      const float den = dens[t];
      Os[t * LS + l16] = f32_to_bf16(o0[r] / den);
      Os[t * LS + 16 + l16] = f32_to_bf16(o1[r] / den);
    }
  };

  load_chunk(0, rqA, rkA, rvA);
  if (nchunks > 1) load_chunk(1, rqB, rkB, rvB);
  for (int c = 0; c < nchunks; c += 2) {
    body(c, rqA, rkA, rvA);
    if (c + 1 < nchunks) body(c + 1, rqB, rkB, rvB);
  }
  __syncthreads();
  {
    const int row = tid >> 2, part = (tid & 3) * 8;
    const int64_t o_off = base + ((int64_t)(nchunks - 1) * LC + row) * LDV + j0 + part;
    nt_store16(a.o + o_off, *reinterpret_cast<const uint4 *>(Os + row * LS + part));
  }
}
