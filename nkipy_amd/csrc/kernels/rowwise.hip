// Fused elementwise + row-reduction kernels (gfx950).
//
//   softmax over the last axis:  y = exp(x - max_row) / sum_row(exp(x - max_row))
//     -- the NumPy composition of softmax_kernel (README.md:125-128,
//        tests/kernels/softmax.py:7-10) and its fp32-upcast variant
//        (examples/models/qwen3_embedding/kernels/softmax.py:4-8).
//   residual + RMSNorm:  h = x (+ r);  y = h / sqrt(mean(h^2) + eps) * w
//     -- rmsnorm_kernel (examples/models/qwen3/kernels/rmsnorm.py:4-21)
//        applied to z = x + h1 (examples/models/qwen3/kernels/transformer_layer.py:60),
//        and the 1/sqrt form of tests/kernels/llama_decoder_dynamo.py:95-107.
//
// Layout: rows of `n` contiguous elements, row-major, one workgroup per row.
// The register variants hold the whole row in VGPRs (CHUNKS x 8 elements per
// thread): every 16-byte streaming (nontemporal) load of the row is issued
// before any arithmetic, so a thread's requests are all in flight together,
// and each input byte is read from HBM once.  The loop variants take any n
// and re-read the row (fallback only).
// Arithmetic is fp32 whatever the storage type.  The register softmax takes
// e^x from the hardware 2^t with the rounding error of t = x log2 e folded
// back in (exp_acc, about two ulp), so fp32 softmax stays within 1e-5 of
// NumPy; the loop fallback calls libm expf.  When the traced softmax runs
// in the 16-bit input type itself (SMX_ROUND_OPS: bf16 or fp16 x - max,
// exp, sum and divide, as softmax_kernel computes on bf16 scores), each
// of those results is rounded to that type as the traced code rounds it:
// d = r(x - max), e = r(exp d), s = r(sum e) with an fp32 sum,
// y = r(e / s).

#include "common.h"

using namespace nk;

struct SoftmaxArgs {
  const void *x;
  void *y;
  int64_t rows;
  int32_t n;
  int32_t flags;
};
enum { SMX_ROUND_OPS = 1 };

// x rounded to the storage type T (fp32: unchanged)
template <typename T>
__device__ __forceinline__ float round_as(float x) {
  if constexpr (sizeof(T) == 4) {
    return x;
  } else {
    T t;
    Elt<T>::store(&t, 0, x);
    return Elt<T>::load(&t, 0);
  }
}

// Loads go through the cache; NTS selects streaming stores (2-byte and
// mixed types).  With each thread's 8 elements contiguous, fp32 measured on
// (2048, 4096) (us, cached / streaming loads): one wave x 8 chunks with
// cached stores 13.8 / 14.4, with streaming stores 18.8 / 18.6.
// The row is addressed through buffer resources of exactly n elements: the
// chunks past its end load zeros and drop their stores, and are left out of
// the max and the sum by a select, so no memory access sits behind a branch
// (the compiler then waits for each load only where its chunk is used).
// fp32 -> fp32 rows take a split layout instead: the 16-byte pieces of a
// thread's chunks lie BLOCK pieces apart, so each load / store instruction
// covers 64 x 16 contiguous bytes, and both go streaming (nontemporal).
// (With a thread's 32 contiguous bytes per chunk, each instruction covers
// half of every line it touches, and a streaming load then misses the half
// the next instruction wants: that is why the loads above stay cached.)
// Softmax is elementwise after its two reductions, so which elements a
// thread holds does not matter; a piece is wholly inside or past the row
// (n is a multiple of 8).  Measured on (2048, 4096) fp32, one wave x 8
// chunks: 13.8 us with the contiguous layout and cached access, 11.5 us
// split and streaming.
template <typename TI, typename TO, int BLOCK, int CHUNKS, bool NTS = true>
__device__ __forceinline__ void softmax_reg_body(const SoftmaxArgs &a) {
  constexpr bool SPLIT = sizeof(TI) == 4 && sizeof(TO) == 4;
  __shared__ float red[BLOCK / 64];
  const int64_t row = blockIdx.x;
  const int n = a.n;
  const auto xr = buf_rsrc(reinterpret_cast<const TI *>(a.x) + row * n, (uint32_t)n * sizeof(TI));
  const auto yr = buf_rsrc(reinterpret_cast<TO *>(a.y) + row * n, (uint32_t)n * sizeof(TO));
  const int tid = threadIdx.x;
  // element offset of half h (4 elements) of chunk c in the split layout
  auto spl = [&](int c, int h) __attribute__((always_inline)) { return ((2 * c + h) * BLOCK + tid) * 4; };
  Raw8<TI> raw[CHUNKS];
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    if constexpr (SPLIT) {
#pragma unroll
      for (int h = 0; h < 2; ++h) raw[c].w[h] = buf_ld16<true>(xr, spl(c, h) * 4);
    } else {
      raw[c].template load_buf<false>(xr, (c * BLOCK + tid) * 8 * sizeof(TI));
    }
  }
  // whether each half (split layout) or the chunk (otherwise) lies inside the row
  auto inside = [&](int c, int j) __attribute__((always_inline)) {
    return SPLIT ? spl(c, j >> 2) < n : (c * BLOCK + tid) * 8 < n;
  };
  float v[CHUNKS][8];
  float m = -INFINITY;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    decode8(raw[c], v[c]);
    float mc = inside(c, 0) ? v[c][0] : -INFINITY;
#pragma unroll
    for (int j = 1; j < 8; ++j) mc = fmaxf(mc, inside(c, j) ? v[c][j] : -INFINITY);
    m = fmaxf(m, mc);
  }
  m = block_max<BLOCK>(m, red);
  // uniform: every thread rounds the same steps
  const bool rnd = (a.flags & SMX_ROUND_OPS) != 0;
  auto r = [&](float x) __attribute__((always_inline)) { return rnd ? round_as<TI>(x) : x; };
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    float sc = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[c][j] = r(exp_acc(r(v[c][j] - m)));
      sc += inside(c, j) ? v[c][j] : 0.f;
    }
    s += sc;
  }
  s = r(block_sum<BLOCK>(s, red));
  const float inv_s = 1.0f / s;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[c][j] = r(div_rn_finite(v[c][j], s, inv_s));
    Raw8<TO> o;
    encode8(v[c], o);
    if constexpr (SPLIT) {
#pragma unroll
      for (int h = 0; h < 2; ++h) buf_st16<true>(yr, spl(c, h) * 4, o.w[h]);
    } else {
      o.template store_buf<NTS>(yr, (c * BLOCK + tid) * 8 * sizeof(TO));
    }
  }
}

template <typename TI, typename TO, int BLOCK>
__device__ __forceinline__ void softmax_loop_body(const SoftmaxArgs &a) {
  __shared__ float red[BLOCK / 64];
  const int64_t row = blockIdx.x;
  const int n = a.n;
  const TI *x = reinterpret_cast<const TI *>(a.x) + row * n;
  TO *y = reinterpret_cast<TO *>(a.y) + row * n;
  float m = -INFINITY;
  for (int i = threadIdx.x; i < n; i += BLOCK) m = fmaxf(m, Elt<TI>::load(x, i));
  m = block_max<BLOCK>(m, red);
  const bool rnd = (a.flags & SMX_ROUND_OPS) != 0;
  auto r = [&](float v) { return rnd ? round_as<TI>(v) : v; };
  float s = 0.f;
  for (int i = threadIdx.x; i < n; i += BLOCK) s += r(expf(r(Elt<TI>::load(x, i) - m)));
  s = r(block_sum<BLOCK>(s, red));
  for (int i = threadIdx.x; i < n; i += BLOCK)
    Elt<TO>::store(y, i, r(r(expf(r(Elt<TI>::load(x, i) - m))) / s));
}

#define NK_SOFTMAX_REG(TI, TO, tin, ton, B, C)                                       \
  extern "C" __global__ __launch_bounds__(B) void nk_softmax_reg_##tin##_##ton##_b##B##_c##C( \
      SoftmaxArgs a) {                                                               \
    softmax_reg_body<TI, TO, B, C, (B > 64)>(a);                                     \
  }
#define NK_SOFTMAX_LOOP(TI, TO, tin, ton)                                             \
  extern "C" __global__ __launch_bounds__(256) void nk_softmax_loop_##tin##_##ton(     \
      SoftmaxArgs a) {                                                               \
    softmax_loop_body<TI, TO, 256>(a);                                               \
  }

#define NK_SOFTMAX_ALL(TI, TO, tin, ton) \
  NK_SOFTMAX_REG(TI, TO, tin, ton, 64, 1)  \
  NK_SOFTMAX_REG(TI, TO, tin, ton, 64, 8)  \
  NK_SOFTMAX_REG(TI, TO, tin, ton, 128, 4) \
  NK_SOFTMAX_REG(TI, TO, tin, ton, 256, 1) \
  NK_SOFTMAX_REG(TI, TO, tin, ton, 256, 2) \
  NK_SOFTMAX_REG(TI, TO, tin, ton, 512, 1) \
  NK_SOFTMAX_REG(TI, TO, tin, ton, 256, 4) \
  NK_SOFTMAX_REG(TI, TO, tin, ton, 512, 4) \
  NK_SOFTMAX_LOOP(TI, TO, tin, ton)

NK_SOFTMAX_ALL(float, float, f32, f32)
NK_SOFTMAX_ALL(bf16, bf16, bf16, bf16)
NK_SOFTMAX_ALL(bf16, float, bf16, f32)
NK_SOFTMAX_ALL(float, bf16, f32, bf16)
NK_SOFTMAX_ALL(f16, f16, f16, f16)

// ---------------------------------------------------------------------------
// Residual + RMSNorm
// ---------------------------------------------------------------------------
struct RmsNormArgs {
  const void *x;
  const void *r;  // residual (flag NK_RMS_RES)
  const void *w;  // weight   (flag NK_RMS_W)
  void *y;
  void *h;        // residual sum out (flag NK_RMS_WRITE_H)
  int64_t rows;
  int32_t n;
  float eps;
  int32_t flags;
  int32_t pad;
};

enum {
  NK_RMS_RES = 1,        // h = x + r
  NK_RMS_ROUND_H = 2,    // round h to the storage type before use (bf16 add)
  NK_RMS_WRITE_H = 4,    // also store h
  NK_RMS_MUL_RECIP = 8,  // y = h * (1/sqrt(.)) instead of h / sqrt(.)
  NK_RMS_W = 16,         // multiply by weight
};

template <typename T>
__device__ __forceinline__ float round_to(float v);
template <> __device__ __forceinline__ float round_to<float>(float v) { return v; }
template <> __device__ __forceinline__ float round_to<bf16>(float v) {
  return bf16_to_f32(f32_to_bf16(v));
}
template <> __device__ __forceinline__ float round_to<f16>(float v) {
  return f16_to_f32(f32_to_f16(v));
}

// RES (residual present) is a template parameter so that the residual loads
// are issued together with the x loads, not behind a runtime branch.  With
// a residual the loads stream (nontemporal), without one they go through the
// cache: bf16 (8192, 4096) measured 33.8 us streaming / 35.9 us cached with
// a residual, 24.0 us / 20.9 us without.  Rows
// are addressed through buffer resources of exactly n elements: chunks past
// the end load zeros (adding nothing to the sum of squares) and drop their
// stores, so no memory access sits behind a branch.
template <typename T, int BLOCK, int CHUNKS, bool RES>
__device__ __forceinline__ void rmsnorm_reg_body(const RmsNormArgs &a) {
  __shared__ float red[BLOCK / 64];
  const int64_t row = blockIdx.x;
  const int n = a.n;
  const int flags = a.flags;
  const uint32_t rb = (uint32_t)n * sizeof(T);
  const auto xr = buf_rsrc(reinterpret_cast<const T *>(a.x) + row * n, rb);
  const auto rr_ = buf_rsrc(RES ? reinterpret_cast<const T *>(a.r) + row * n : nullptr, RES ? rb : 0);
  const auto wr = buf_rsrc(a.w, (flags & NK_RMS_W) ? rb : 0);
  const auto yr = buf_rsrc(reinterpret_cast<T *>(a.y) + row * n, rb);
  const auto hr = buf_rsrc((flags & NK_RMS_WRITE_H) ? reinterpret_cast<T *>(a.h) + row * n : nullptr,
                           (flags & NK_RMS_WRITE_H) ? rb : 0);
  const int tid = threadIdx.x;
  Raw8<T> xv[CHUNKS], rv_[CHUNKS], wraw[CHUNKS];
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const uint32_t off = (c * BLOCK + tid) * 8 * sizeof(T);
    xv[c].template load_buf<RES>(xr, off);
    if (RES) rv_[c].template load_buf<RES>(rr_, off);
  }
  // the weight (the same row for every workgroup, cache-resident) is
  // fetched with the row, not after the reduction: no second memory round
  // trip between the sum and the stores
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c)
    if (flags & NK_RMS_W) wraw[c].template load_buf<false>(wr, (c * BLOCK + tid) * 8 * sizeof(T));
  float v[CHUNKS][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    decode8(xv[c], v[c]);
    if (RES) {
      float rv[8];
      decode8(rv_[c], rv);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[c][j] += rv[j];
      if (flags & NK_RMS_ROUND_H) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[c][j] = round_to<T>(v[c][j]);
      }
      if (flags & NK_RMS_WRITE_H) {
        Raw8<T> o;
        encode8(v[c], o);
        o.template store_buf<true>(hr, (c * BLOCK + tid) * 8 * sizeof(T));
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += v[c][j] * v[c][j];
  }
  ss = block_sum<BLOCK>(ss, red);
  const float ms = ss / (float)n;
  const float s = sqrtf(ms + a.eps);
  const float inv = 1.0f / s;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const uint32_t off = (c * BLOCK + tid) * 8 * sizeof(T);
    float wv[8];
    if (flags & NK_RMS_W) decode8(wraw[c], wv);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float q = (flags & NK_RMS_MUL_RECIP) ? v[c][j] * inv : div_rn(v[c][j], s, inv);
      if (flags & NK_RMS_W) q = q * wv[j];
      v[c][j] = q;
    }
    Raw8<T> o;
    encode8(v[c], o);
    o.template store_buf<true>(yr, off);
  }
}

template <typename T, int BLOCK>
__device__ __forceinline__ void rmsnorm_loop_body(const RmsNormArgs &a) {
  __shared__ float red[BLOCK / 64];
  const int64_t row = blockIdx.x;
  const int n = a.n;
  const int flags = a.flags;
  const T *x = reinterpret_cast<const T *>(a.x) + row * n;
  const T *r = reinterpret_cast<const T *>(a.r) + row * n;
  const T *w = reinterpret_cast<const T *>(a.w);
  T *y = reinterpret_cast<T *>(a.y) + row * n;
  T *h = reinterpret_cast<T *>(a.h) + row * n;
  float ss = 0.f;
  for (int i = threadIdx.x; i < n; i += BLOCK) {
    float v = Elt<T>::load(x, i);
    if (flags & NK_RMS_RES) {
      v += Elt<T>::load(r, i);
      if (flags & NK_RMS_ROUND_H) v = round_to<T>(v);
    }
    ss += v * v;
  }
  ss = block_sum<BLOCK>(ss, red);
  const float ms = ss / (float)n;
  const float s = sqrtf(ms + a.eps);
  const float inv = 1.0f / s;
  for (int i = threadIdx.x; i < n; i += BLOCK) {
    float v = Elt<T>::load(x, i);
    if (flags & NK_RMS_RES) {
      v += Elt<T>::load(r, i);
      if (flags & NK_RMS_ROUND_H) v = round_to<T>(v);
      if (flags & NK_RMS_WRITE_H) Elt<T>::store(h, i, v);
    }
    float q = (flags & NK_RMS_MUL_RECIP) ? v * inv : v / s;
    if (flags & NK_RMS_W) q = q * Elt<T>::load(w, i);
    Elt<T>::store(y, i, q);
  }
}

// Register variants: nk_rmsnorm_reg_<t>_b<BLOCK>_c<CHUNKS> (no residual) and
// nk_rmsnorm_res_<t>_b<BLOCK>_c<CHUNKS> (residual).
#define NK_RMS_REG(T, tn, B, C)                                                       \
  extern "C" __global__ __launch_bounds__(B) void nk_rmsnorm_reg_##tn##_b##B##_c##C(   \
      RmsNormArgs a) {                                                                \
    rmsnorm_reg_body<T, B, C, false>(a);                                              \
  }                                                                                   \
  extern "C" __global__ __launch_bounds__(B) void nk_rmsnorm_res_##tn##_b##B##_c##C(   \
      RmsNormArgs a) {                                                                \
    rmsnorm_reg_body<T, B, C, true>(a);                                               \
  }
#define NK_RMS_LOOP(T, tn)                                                           \
  extern "C" __global__ __launch_bounds__(256) void nk_rmsnorm_loop_##tn(RmsNormArgs a) { \
    rmsnorm_loop_body<T, 256>(a);                                                    \
  }
#define NK_RMS_ALL(T, tn) \
  NK_RMS_REG(T, tn, 64, 1)  \
  NK_RMS_REG(T, tn, 128, 4) \
  NK_RMS_REG(T, tn, 256, 1) \
  NK_RMS_REG(T, tn, 256, 2) \
  NK_RMS_REG(T, tn, 512, 1) \
  NK_RMS_REG(T, tn, 256, 4) \
  NK_RMS_REG(T, tn, 512, 4) \
  NK_RMS_LOOP(T, tn)

NK_RMS_ALL(float, f32)
NK_RMS_ALL(bf16, bf16)
NK_RMS_ALL(f16, f16)
