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
