// Rotary position embedding, split-half form, bf16 in / bf16 out.
//
//   out[.., :D/2] = x0 * cos - x1 * sin
//   out[.., D/2:] = x0 * sin + x1 * cos        x0 = x[.., :D/2], x1 = x[.., D/2:]
//
// as written in examples/models/qwen3/kernels/rope.py:23-48 (tables indexed
// by position s and frequency d, broadcast over batch and heads).  Each
// product, sum and difference is rounded to fp32 separately (no fused
// multiply-add), as NumPy evaluates it; the result is rounded to bf16 once.
//
// x is read through strides (b, s, h) with d contiguous, so q and k are read
// straight out of a fused QKV projection.  One thread handles 8 frequencies
// of one (b, s, h) row: two 16-byte loads of x, 32-byte loads of each table
// (L2-resident: S x D/2 fp32), two 16-byte stores.

#include "common.h"

using namespace nk;

struct RopeArgs {
  const uint16_t *x;
  const float *cos_t;
  const float *sin_t;
  uint16_t *out;
  int64_t x_sb, x_ss, x_sh;  // element strides of x over (b, s, h)
  int64_t o_sb, o_ss, o_sh;  // element strides of out
  int64_t x_half;            // element offset of x1 from x0
  int64_t t_ss;              // table stride over s (frequency contiguous)
  int64_t groups;            // B * S * H * (half / 8)
  int32_t S, H, half, nthreads;
};

__device__ __forceinline__ void unpack8(uint4 r, float *f) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ uint4 pack8(const float *f) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

extern "C" __global__ __launch_bounds__(256) void nk_rope_bf16(RopeArgs a) {
  const int per_row = a.half >> 3;
  for (int64_t gi = (int64_t)blockIdx.x * 256 + threadIdx.x; gi < a.groups; gi += a.nthreads) {
    const int j = (int)(gi % per_row);
    const int64_t row = gi / per_row;
    const int h = (int)(row % a.H);
    const int64_t bs = row / a.H;
    const int s = (int)(bs % a.S);
    const int64_t b = bs / a.S;
    const int64_t xo = b * a.x_sb + s * a.x_ss + h * a.x_sh + 8 * j;
    const uint4 r0 = *reinterpret_cast<const uint4 *>(a.x + xo);
    const uint4 r1 = *reinterpret_cast<const uint4 *>(a.x + xo + a.x_half);
    const float *cp = a.cos_t + (int64_t)s * a.t_ss + 8 * j;
    const float *sp = a.sin_t + (int64_t)s * a.t_ss + 8 * j;
    const float4 c0 = *reinterpret_cast<const float4 *>(cp);
    const float4 c1 = *reinterpret_cast<const float4 *>(cp + 4);
    const float4 s0 = *reinterpret_cast<const float4 *>(sp);
    const float4 s1 = *reinterpret_cast<const float4 *>(sp + 4);
    const float c[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    float x0[8], x1[8], y0[8], y1[8];
    unpack8(r0, x0);
    unpack8(r1, x1);
    {
      // separate roundings of each product and of the sum / difference
#pragma clang fp contract(off)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        y0[i] = x0[i] * c[i] - x1[i] * sn[i];
        y1[i] = x0[i] * sn[i] + x1[i] * c[i];
      }
    }
    const int64_t oo = b * a.o_sb + s * a.o_ss + h * a.o_sh + 8 * j;
    *reinterpret_cast<uint4 *>(a.out + oo) = pack8(y0);
    *reinterpret_cast<uint4 *>(a.out + oo + a.half) = pack8(y1);
  }
}

// ---------------------------------------------------------------------------
// Per-head RMSNorm and rotary embedding in bf16 steps: the prologue of
// examples/models/qwen3/kernels/attention.py:79-97 (q / k RMSNorm over
// head_dim, then rope.py:4-48 with the cos / sin tables cast to bf16 and
// taken at the current positions), where every product, sum and difference
// is a bf16 array:
//
//   y = bf16(h / sqrt(mean(h*h) + eps) * w)             (fp32 arithmetic)
//   out[.., :D/2] = bf16(bf16(y0 * c) - bf16(y1 * s))
//   out[.., D/2:] = bf16(bf16(y0 * s) + bf16(y1 * c))   y0 / y1 = halves of y
//
// One head row of D <= 128 elements per 16-lane DPP row of a wavefront:
// lane l holds elements 8l .. 8l+7, so the sum of squares is formed exactly
// as the RMSNorm row kernel forms it for a row of D elements (each lane's
// eight squares in order, then the same four DPP steps within the 16 lanes,
// lane 0's sum): the normalised values equal that kernel's bit for bit.
// Lane l of the first half and lane l + D/16 of the second exchange their
// values (one ds_bpermute each), then both apply the rotation to the same
// eight frequencies.  Up to two targets (q and k heads) share the tables; a
// workgroup (16 rows) serves one target, so their fields are uniform.
// Tables are fp32 (rounded to bf16 as they are read: the traced astype) or
// bf16, indexed [row * t_row + s * t_ss + f]; row is the runtime position
// pos[0] (negative counts from the end, then clamped into the table, as the
// gather kernel treats an index) or 0.
// A third target copies its rows unchanged (HR_COPY: the v heads).  A target
// with o_sp != 0 writes its rows at the runtime position of the output's
// position axis (the cache write cache[:, pos] = k of one decode token): the
// scatter kernel's rule, negative counts from the end and a position outside
// the o_rows positions drops the store.
// HR_PLANES: x addresses the fp32 partial sums of the projection that
// produced the rows (nplanes planes of `plane` elements, the layout of the
// few-row projections' workspace) instead of its bf16 output; the planes
// are added as nk_gemv_out_bf16 adds them (plane p into sum p mod 4 in
// order from 0, then (s0 + s1) + (s2 + s3), then + 0 and the bf16 rounding),
// so the rows equal that kernel's output bit for bit and its launch is
// saved.
// ---------------------------------------------------------------------------
struct HeadRopeTarget {
  const uint16_t *x;         // bf16 input rows, d contiguous
  uint16_t *out;             // bf16 rotated rows
  const uint16_t *w;         // bf16 norm weight (D elements) or null
  int64_t x_sb, x_ss, x_sh;  // element strides of x over (b, s, h)
  int64_t o_sb, o_ss, o_sh;  // element strides of out
  int64_t x_half;            // element offset of the second half in an input row
  int64_t rows;              // B * S * H
  int64_t blocks;            // workgroups serving this target
  int64_t o_sp, o_rows;      // runtime output position: element stride, positions
  float eps;
  int32_t H, flags, pad;
};

struct HeadRopeArgs {
  HeadRopeTarget t[3];
  const void *cos_t;
  const void *sin_t;
  const int32_t *pos;  // runtime table row, or null
  int64_t t_row;       // table elements per runtime row
  int64_t t_ss;        // table element stride over s
  int64_t t_rows;      // table rows (runtime row clamp)
  int32_t S, D, tflags, pad;
  int64_t plane;       // HR_PLANES: elements per partial-sum plane
  int32_t nplanes;     // HR_PLANES: planes (1 .. HR_MAX_PLANES)
  int32_t pad2;
};

enum { HR_NORM = 1, HR_MUL_RECIP = 2, HR_W = 4, HR_COPY = 8, HR_PLANES = 16 };  // per target
constexpr int HR_MAX_PLANES = 32;
enum { HR_TABLE_F32 = 1 };

__device__ __forceinline__ float rbf(float v) { return bf16_to_f32(f32_to_bf16(v)); }

extern "C" __global__ __launch_bounds__(256) void nk_head_rope_bf16(HeadRopeArgs a) {
  const int tid = threadIdx.x;
  const int lane = tid & 15;
  const int64_t bid = blockIdx.x, b0 = a.t[0].blocks, b01 = b0 + a.t[1].blocks;
  const int tg = bid >= b01 ? 2 : (bid >= b0 ? 1 : 0);
  // uniform per workgroup: scalar selects, no indexing of the argument array
#define HR_SEL(f) (tg == 2 ? a.t[2].f : (tg == 1 ? a.t[1].f : a.t[0].f))
  const uint16_t *x = HR_SEL(x);
  uint16_t *out = HR_SEL(out);
  const uint16_t *w = HR_SEL(w);
  const int64_t x_sb = HR_SEL(x_sb), x_ss = HR_SEL(x_ss), x_sh = HR_SEL(x_sh), x_half = HR_SEL(x_half);
  const int64_t o_sb = HR_SEL(o_sb), o_ss = HR_SEL(o_ss), o_sh = HR_SEL(o_sh), nrows = HR_SEL(rows);
  const int64_t o_sp = HR_SEL(o_sp), o_rows = HR_SEL(o_rows);
  const float eps = HR_SEL(eps);
  const int H = HR_SEL(H), flags = HR_SEL(flags);
#undef HR_SEL
  const int64_t row = (bid - (tg == 2 ? b01 : (tg == 1 ? b0 : 0))) * 16 + (tid >> 4);

  const int D = a.D, half = D >> 1, hl = D >> 4;  // hl: lanes per half row
  const bool second = lane >= hl;
  const bool live = row < nrows && lane < 2 * hl;
  // rows < 2^31 (checked by the launcher): 32-bit index arithmetic
  const uint32_t r = live ? (uint32_t)row : 0u;
  const int h = (int)(r % (uint32_t)H);
  const uint32_t bs = r / (uint32_t)H;
  const int s = (int)(bs % (uint32_t)a.S);
  const int64_t b = bs / (uint32_t)a.S;
  const int f0 = live ? 8 * (second ? lane - hl : lane) : 0;  // first frequency of the lane
  const int64_t col = (second ? half : 0) + f0;                // element of the row

  // every load first: x chunk (or its partial sums), weight chunk, table chunks
  const int64_t xo = live ? b * x_sb + s * x_ss + h * x_sh + (second ? x_half : 0) + f0 : 0;
  float v[8];
  if (flags & HR_PLANES) {
    const float *xp = reinterpret_cast<const float *>(x) + xo;
    const int np = a.nplanes;
    float g[4][8];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) g[j][e] = 0.f;
#pragma unroll
    for (int s0 = 0; s0 < HR_MAX_PLANES; s0 += 4) {
      if (s0 >= np) break;  // uniform
      float4 q[4][2];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 *pp = reinterpret_cast<const float4 *>(xp + (int64_t)min(s0 + j, np - 1) * a.plane);
        q[j][0] = pp[0];
        q[j][1] = pp[1];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (s0 + j < np) {
          const float qv[8] = {q[j][0].x, q[j][0].y, q[j][0].z, q[j][0].w,
                               q[j][1].x, q[j][1].y, q[j][1].z, q[j][1].w};
#pragma unroll
          for (int e = 0; e < 8; ++e) g[j][e] += qv[e];
        }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = rbf(((g[0][e] + g[1][e]) + (g[2][e] + g[3][e])) + 0.f);
  } else {
    unpack8(*reinterpret_cast<const uint4 *>(x + xo), v);
  }
  uint4 wr = make_uint4(0, 0, 0, 0);
  if (flags & HR_W) wr = *reinterpret_cast<const uint4 *>(w + (live ? col : 0));
  int64_t trow = 0;
  if (a.pos != nullptr) {
    int64_t j = a.pos[0];
    if (j < 0) j += a.t_rows;
    trow = j < 0 ? 0 : (j >= a.t_rows ? a.t_rows - 1 : j);
  }
  const int64_t to = trow * a.t_row + (int64_t)s * a.t_ss + f0;
  float c[8], sn[8];
  if (a.tflags & HR_TABLE_F32) {
    const float4 *cp = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(a.cos_t) + to);
    const float4 *sp = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(a.sin_t) + to);
    const float4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
    const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      c[i] = rbf(cv[i]);
      sn[i] = rbf(sv[i]);
    }
  } else {
    unpack8(*reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(a.cos_t) + to), c);
    unpack8(*reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(a.sin_t) + to), sn);
  }

#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = live ? v[j] : 0.f;
  if (flags & HR_NORM) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += v[j] * v[j];
    ss = ss + dpp<0xB1>(ss);
    ss = ss + dpp<0x4E>(ss);
    ss = ss + dpp<0x124>(ss);
    ss = ss + dpp<0x128>(ss);
    ss = __shfl(ss, (tid & 63) & ~15);
    const float ms = ss / (float)D;
    const float sd = sqrtf(ms + eps);
    const float inv = 1.0f / sd;
    float wv[8];
    unpack8(wr, wv);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float q = (flags & HR_MUL_RECIP) ? v[j] * inv : div_rn(v[j], sd, inv);
      if (flags & HR_W) q = q * wv[j];
      v[j] = rbf(q);
    }
  }
  // partner lane: the other half of the same frequencies
  const int src = ((tid & 63) & ~15) + (second ? lane - hl : lane + hl);
  float y[8];
  if (flags & HR_COPY) {
#pragma unroll
    for (int j = 0; j < 8; ++j) y[j] = v[j];
  } else {
#pragma clang fp contract(off)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float p = __shfl(v[j], src);
      // first half: y0 c - y1 s; second half: y0 s + y1 c (own value y1)
      const float own = rbf(v[j] * c[j]);
      const float oth = rbf(p * sn[j]);
      y[j] = rbf(second ? oth + own : own - oth);
    }
  }
  int64_t oo = b * o_sb + s * o_ss + h * o_sh + col;
  bool store = live;
  if (o_sp != 0) {
    int64_t j = a.pos[0];
    if (j < 0) j += o_rows;
    store = store && j >= 0 && j < o_rows;
    oo += (store ? j : 0) * o_sp;
  }
  if (store) *reinterpret_cast<uint4 *>(out + oo) = pack8(y);
}
