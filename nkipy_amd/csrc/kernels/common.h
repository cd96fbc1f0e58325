// Shared device helpers for the NKIPy gfx950 kernels: storage types,
// bf16 / fp8-e4m3fn / fp16 conversions, 16-byte vector access and
// wavefront / workgroup reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define NK_DEVICE __device__ __forceinline__

namespace nk {

// ---------------------------------------------------------------------------
// Storage types.  Tensors cross the C ABI as raw bytes; kernels reinterpret
// them with these tags.  bf16 and fp8 are stored as their bit patterns.
// ---------------------------------------------------------------------------
struct bf16 { uint16_t bits; };
struct f16 { uint16_t bits; };
struct e4m3 { uint8_t bits; };  // OCP float8 E4M3FN: bias 7, no inf, 0x7f/0xff NaN

NK_DEVICE float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// Round-to-nearest-even float -> bf16 with the hardware conversion
// (v_cvt_pk_bf16_f32): for every non-NaN input it equals the closed form
// "add 0x7fff plus the kept LSB, truncate"; a NaN stays a (quiet) NaN.  The
// branch-free instruction replaces a per-element NaN test that compiled to
// divergent branches.
NK_DEVICE uint16_t f32_to_bf16(float f) {
  const __bf16 b = (__bf16)f;
  uint16_t h;
  __builtin_memcpy(&h, &b, 2);
  return h;
}

// Correctly rounded a / b from rb = RN(1 / b), for a row of quotients that
// share one divisor: q = RN(a * rb) is within one ulp of a / b, the fma
// residual a - q * b and one fma correction then give RN(a / b) (Markstein,
// IBM J. Res. Dev. 34(1), 1990).  Three instructions instead of the
// scale / reciprocal / fixup sequence of a full division.  A non-finite
// correction (b infinite, a infinite or NaN) falls back to q, which then
// equals the IEEE quotient.
NK_DEVICE float div_rn(float a, float b, float rb) {
  const float q = a * rb;
  const float r = __builtin_fmaf(-q, b, a);
  const float c = __builtin_fmaf(r, rb, q);
  return __builtin_isfinite(c) ? c : q;
}

// The same correction without the fallback, for quotients known to stay
// finite (a finite, b finite and >= 1).
NK_DEVICE float div_rn_finite(float a, float b, float rb) {
  const float q = a * rb;
  const float r = __builtin_fmaf(-q, b, a);
  return __builtin_fmaf(r, rb, q);
}

// e^x from the hardware 2^t (v_exp_f32, about one ulp) at t = RN(x * L),
// L = RN(log2 e), corrected by the part of x * log2 e that t leaves out:
// e = (x * L - t) + x * (log2 e - L), the first term exact from one fma, so
// x * log2 e = t + e to within |x| * 2^-48, and 2^(t + e) = 2^t (1 + e ln 2)
// to within e^2 < 1e-10.  Within about two ulp of e^x over the normal range
// (the product t alone would lose up to |x| * 6e-8 relative).  Inputs below
// -200 are clamped, where the result underflows to 0 either way, so -inf
// gives 0 and NaN stays NaN.
NK_DEVICE float exp_acc(float x) {
  constexpr float L = 1.44269502f;        // RN(log2 e)
  constexpr float LLO = 1.925963033e-8f;  // log2 e - L
  constexpr float LN2 = 0.693147182f;
  x = x < -200.f ? -200.f : x;
  const float t = x * L;
  const float e = __builtin_fmaf(x, LLO, __builtin_fmaf(x, L, -t));
  const float p = __builtin_amdgcn_exp2f(t);
  return __builtin_fmaf(p, e * LN2, p);
}

NK_DEVICE float f16_to_f32(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;
}
NK_DEVICE uint16_t f32_to_f16(float f) {
  _Float16 v = (_Float16)f;
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

// E4M3FN decode: sign, 4-bit exponent (bias 7), 3-bit mantissa; exponent 0
// is subnormal (2^-6 * m/8); 0x7f / 0xff are NaN; no infinities.
NK_DEVICE float e4m3_to_f32(uint8_t b) {
  uint32_t s = (uint32_t)(b & 0x80u) << 24;
  uint32_t e = (b >> 3) & 0xfu;
  uint32_t m = b & 0x7u;
  if ((b & 0x7fu) == 0x7fu) return __uint_as_float(0x7fc00000u | s);
  if (e == 0) {
    float v = (float)m * 0.001953125f;  // m/8 * 2^-6
    return __uint_as_float(__float_as_uint(v) | s);
  }
  return __uint_as_float(s | ((e + 120u) << 23) | (m << 20));
}

// 8 fp8 E4M3FN (one 64-bit word) -> 8 bf16, exact (3 mantissa bits fit in
// bf16's 7; E4M3 subnormals are bf16 normals).  gfx950's
// v_cvt_scalef32_pk_bf16_fp8 decodes two OCP E4M3FN codes per instruction;
// the scale operand 1.0 leaves the values unscaled.
typedef __bf16 nk_bf16x2 __attribute__((ext_vector_type(2)));
NK_DEVICE uint32_t bf16x2_bits(nk_bf16x2 v) {
  uint32_t u;
  __builtin_memcpy(&u, &v, 4);
  return u;
}
// Two floats -> packed bf16 pair (lo in bits 0..15) with the hardware
// round-to-nearest-even conversion (v_cvt_pk_bf16_f32); NaN inputs give a
// quiet NaN.
NK_DEVICE uint32_t pack_bf16x2(float lo, float hi) {
  const nk_bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return bf16x2_bits(v);
}
NK_DEVICE uint4 e4m3x8_to_bf16x8(uint2 q) {
  return make_uint4(bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q.x, 1.0f, false)),
                    bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q.x, 1.0f, true)),
                    bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q.y, 1.0f, false)),
                    bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q.y, 1.0f, true)));
}

// 128-bit nontemporal (streaming) global access: data read or written once
// per kernel bypasses cache retention, which measurably raises achieved HBM
// bandwidth for the row kernels.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
NK_DEVICE uint4 nt_load16(const void *p) {
  u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return make_uint4(t.x, t.y, t.z, t.w);
}
NK_DEVICE void nt_store16(void *p, uint4 v) {
  u32x4 t = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(t, reinterpret_cast<u32x4 *>(p));
}

// Load / store of one element, converting to / from float.
template <typename T> struct Elt;
template <> struct Elt<float> {
  static NK_DEVICE float load(const float *p, long i) { return p[i]; }
  static NK_DEVICE void store(float *p, long i, float v) { p[i] = v; }
};
template <> struct Elt<bf16> {
  static NK_DEVICE float load(const bf16 *p, long i) { return bf16_to_f32(p[i].bits); }
  static NK_DEVICE void store(bf16 *p, long i, float v) { p[i].bits = f32_to_bf16(v); }
};
template <> struct Elt<f16> {
  static NK_DEVICE float load(const f16 *p, long i) { return f16_to_f32(p[i].bits); }
  static NK_DEVICE void store(f16 *p, long i, float v) { p[i].bits = f32_to_f16(v); }
};

// 16-byte global load / store, streaming (nontemporal) when NT.
template <bool NT>
NK_DEVICE uint4 ld16(const void *p) {
  if (NT) return nt_load16(p);
  return *reinterpret_cast<const uint4 *>(p);
}
template <bool NT>
NK_DEVICE void st16(void *p, uint4 v) {
  if (NT) nt_store16(p, v);
  else *reinterpret_cast<uint4 *>(p) = v;
}

// Eight consecutive elements (16 bytes for 2-byte types, 32 bytes for fp32)
// with 128-bit accesses; `p` must be 16-byte aligned.  NT selects streaming
// access for data touched once.
template <typename T> struct Vec8;
template <> struct Vec8<float> {
  template <bool NT = false>
  static NK_DEVICE void load(const float *p, float v[8]) {
    uint4 a = ld16<NT>(p), b = ld16<NT>(p + 4);
    v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y);
    v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
    v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y);
    v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
  }
  template <bool NT = false>
  static NK_DEVICE void store(float *p, const float v[8]) {
    st16<NT>(p, make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]),
                           __float_as_uint(v[2]), __float_as_uint(v[3])));
    st16<NT>(p + 4, make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]),
                               __float_as_uint(v[6]), __float_as_uint(v[7])));
  }
};
template <> struct Vec8<bf16> {
  template <bool NT = false>
  static NK_DEVICE void load(const bf16 *p, float v[8]) {
    uint4 u = ld16<NT>(p);
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  template <bool NT = false>
  static NK_DEVICE void store(bf16 *p, const float v[8]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    st16<NT>(p, make_uint4(w[0], w[1], w[2], w[3]));
  }
};
template <> struct Vec8<f16> {
  template <bool NT = false>
  static NK_DEVICE void load(const f16 *p, float v[8]) {
    uint4 u = ld16<NT>(p);
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = f16_to_f32((uint16_t)(w[i] & 0xffffu));
      v[2 * i + 1] = f16_to_f32((uint16_t)(w[i] >> 16));
    }
  }
  template <bool NT = false>
  static NK_DEVICE void store(f16 *p, const float v[8]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)f32_to_f16(v[2 * i]) | ((uint32_t)f32_to_f16(v[2 * i + 1]) << 16);
    st16<NT>(p, make_uint4(w[0], w[1], w[2], w[3]));
  }
};

// 16-bit element e (0..7) of a 16-byte word holding 8 two-byte values.
NK_DEVICE uint32_t h16_of(const uint4 &v, int e) {
  uint32_t w = (e < 2) ? v.x : (e < 4) ? v.y : (e < 6) ? v.z : v.w;
  return (e & 1) ? (w >> 16) : (w & 0xffffu);
}

// Buffer resource over `bytes` bytes at p: a load past the end reads zeros
// and a store past the end is dropped, so a partial row needs no branch
// around its memory accesses.  NT sets the streaming (nontemporal) policy.
NK_DEVICE __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
typedef unsigned int nk_u32x4 __attribute__((ext_vector_type(4)));
// `soff` is a wave-uniform byte offset (an SGPR operand of the instruction).
template <bool NT>
NK_DEVICE uint4 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff = 0) {
  const nk_u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(r, off, soff, NT ? 2 : 0);
  return make_uint4(q[0], q[1], q[2], q[3]);
}
typedef unsigned int nk_u32x2 __attribute__((ext_vector_type(2)));
NK_DEVICE void buf_st8(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff, uint2 v) {
  const nk_u32x2 q = {v.x, v.y};
  __builtin_amdgcn_raw_buffer_store_b64(q, r, off, soff, 0);
}
template <bool NT>
NK_DEVICE void buf_st16(__amdgpu_buffer_rsrc_t r, uint32_t off, uint4 v) {
  const nk_u32x4 q = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(q, r, off, 0, NT ? 2 : 0);
}

// ---------------------------------------------------------------------------
// LDS DMA (buffer_load_dwordx4 ... lds) issued as inline asm.  The compiler's
// wait insertion does not model it, so it adds no waits of its own for it
// (its alias analysis cannot separate the slots of one LDS array): every
// wait on a move is explicit in the kernel that issues it.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void;
typedef int i32x4_t __attribute__((ext_vector_type(4)));
// buffer resource words over `bytes` bytes at p (raw, untyped): a move past
// the end fills its 16 bytes with zeros and reads no memory
NK_DEVICE i32x4_t rsrc_words(const void *p, int64_t bytes) {
  const uint64_t ad = (uint64_t)p;
  i32x4_t r;
  r[0] = (int)(uint32_t)ad;
  r[1] = (int)(uint32_t)(ad >> 32) & 0xffff;
  r[2] = (int)bytes;
  r[3] = 0x00020000;
  return r;
}
// LDS byte address of a shared-memory array
NK_DEVICE uint32_t lds_addr(const uint8_t *p) { return (uint32_t)(uintptr_t)(lds_void *)p; }
// lane l of the wave fills LDS byte address lds + 16 l (lds wave-uniform)
// from byte offset off of the resource
NK_DEVICE void dma16_asm(i32x4_t r, uint32_t lds, uint32_t off) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :: "v"(off), "s"(r), "s"(m) : "memory", "m0");
}

// Raw form of an 8-element chunk: U 16-byte words (1 for 2-byte types, 2 for
// fp32).  Kernels issue every raw load of a row first, then decode, so all
// of a thread's HBM requests are in flight together.
template <typename T> struct Raw8 {
  static constexpr int U = sizeof(T) * 8 / 16;
  uint4 w[U];
  // chunk at byte offset `off` of a buffer resource (zeros past its end)
  template <bool NT>
  NK_DEVICE void load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
#pragma unroll
    for (int u = 0; u < U; ++u) w[u] = buf_ld16<NT>(r, off + 16 * u);
  }
  template <bool NT>
  NK_DEVICE void store_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) const {
#pragma unroll
    for (int u = 0; u < U; ++u) buf_st16<NT>(r, off + 16 * u, w[u]);
  }
  template <bool NT>
  NK_DEVICE void load(const T *p) {
#pragma unroll
    for (int u = 0; u < U; ++u) w[u] = ld16<NT>(reinterpret_cast<const uint8_t *>(p) + 16 * u);
  }
  template <bool NT>
  NK_DEVICE void store(T *p) const {
#pragma unroll
    for (int u = 0; u < U; ++u) st16<NT>(reinterpret_cast<uint8_t *>(p) + 16 * u, w[u]);
  }
};

NK_DEVICE void decode8(const Raw8<float> &r, float v[8]) {
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    v[4 * u + 0] = __uint_as_float(r.w[u].x);
    v[4 * u + 1] = __uint_as_float(r.w[u].y);
    v[4 * u + 2] = __uint_as_float(r.w[u].z);
    v[4 * u + 3] = __uint_as_float(r.w[u].w);
  }
}
NK_DEVICE void decode8(const Raw8<bf16> &r, float v[8]) {
  uint32_t w[4] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
NK_DEVICE void decode8(const Raw8<f16> &r, float v[8]) {
  uint32_t w[4] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = f16_to_f32((uint16_t)(w[i] & 0xffffu));
    v[2 * i + 1] = f16_to_f32((uint16_t)(w[i] >> 16));
  }
}
NK_DEVICE void encode8(const float v[8], Raw8<float> &r) {
#pragma unroll
  for (int u = 0; u < 2; ++u)
    r.w[u] = make_uint4(__float_as_uint(v[4 * u]), __float_as_uint(v[4 * u + 1]),
                        __float_as_uint(v[4 * u + 2]), __float_as_uint(v[4 * u + 3]));
}
NK_DEVICE void encode8(const float v[8], Raw8<bf16> &r) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
  r.w[0] = make_uint4(w[0], w[1], w[2], w[3]);
}
NK_DEVICE void encode8(const float v[8], Raw8<f16> &r) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = (uint32_t)f32_to_f16(v[2 * i]) | ((uint32_t)f32_to_f16(v[2 * i + 1]) << 16);
  r.w[0] = make_uint4(w[0], w[1], w[2], w[3]);
}

// ---------------------------------------------------------------------------
// Workgroup barrier for LDS hand-offs.  __syncthreads() carries a release
// fence, which also waits for every outstanding global load (vmcnt(0)) and
// so drains a register prefetch issued ahead of the barrier.  This waits only
// for the wave's own LDS operations (lgkmcnt(0)) before s_barrier; the empty
// asm statements keep the compiler from moving memory accesses across it.
// ---------------------------------------------------------------------------
NK_DEVICE void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------
// Reductions.  A wavefront is 64 lanes on CDNA4, in four rows of 16.  Within
// a row, DPP operands (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_ror 4,
// row_ror 8) combine lanes without LDS traffic; the four row results are then
// read with v_readlane.  Every lane must be active.
// ---------------------------------------------------------------------------
template <bool MAX>
NK_DEVICE float red_op(float a, float b) {
  return MAX ? fmaxf(a, b) : a + b;
}
template <int CTRL>
NK_DEVICE float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <bool MAX>
NK_DEVICE float wave_reduce(float v) {
  v = red_op<MAX>(v, dpp<0xB1>(v));
  v = red_op<MAX>(v, dpp<0x4E>(v));
  v = red_op<MAX>(v, dpp<0x124>(v));
  v = red_op<MAX>(v, dpp<0x128>(v));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return red_op<MAX>(red_op<MAX>(r0, r1), red_op<MAX>(r2, r3));
}
NK_DEVICE float wave_sum(float v) { return wave_reduce<false>(v); }
NK_DEVICE float wave_max(float v) { return wave_reduce<true>(v); }

// Workgroup reductions over BLOCK threads (BLOCK a multiple of 64, <= 1024).
// `red` is a __shared__ scratch of at least BLOCK/64 floats; the function
// synchronises before reusing it, so back-to-back calls are safe.
template <int BLOCK, bool MAX>
NK_DEVICE float block_reduce(float v, float *red) {
  v = wave_reduce<MAX>(v);
  if (BLOCK == 64) return v;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  lds_barrier();
  if (lane == 0) red[wid] = v;
  lds_barrier();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < BLOCK / 64; ++i) t = red_op<MAX>(t, red[i]);
  return t;
}
template <int BLOCK>
NK_DEVICE float block_sum(float v, float *red) {
  return block_reduce<BLOCK, false>(v, red);
}
template <int BLOCK>
NK_DEVICE float block_max(float v, float *red) {
  return block_reduce<BLOCK, true>(v, red);
}

}  // namespace nk
