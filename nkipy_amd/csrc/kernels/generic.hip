// Generic fallback kernels for graph nodes no fused pattern covers.
//
// nk_ew_program: one thread per output element evaluates a short register
//   program (loads with arbitrary strides -- broadcast, transpose, slice and
//   reverse are stride patterns -- constants, iota, unary / binary / select /
//   compare ops).  Registers are double; every instruction rounds its result
//   to the dtype of the graph node it implements, so chained ops see the same
//   intermediate roundings as NumPy in the node dtype.
// nk_reduce:   one workgroup per output element, any set of reduced axes.
// nk_dot:      batched C = A * B with arbitrary operand strides, LDS tiles,
//              fp32 accumulation.  Fallback only: the fused GEMM kernels are
//              the fast path.
// nk_gather / nk_scatter: take, take_along_axis, scatter / put along axis.
// nk_cumsum:   sequential scan per line.
//
// Index operands are clamped into range (never a fault on bad indices).

#include "common.h"

using namespace nk;

enum DType : int32_t {
  DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2, DT_E4M3 = 3, DT_I8 = 4, DT_I16 = 5,
  DT_I32 = 6, DT_I64 = 7, DT_U8 = 8, DT_U16 = 9, DT_U32 = 10, DT_U64 = 11,
  DT_BOOL = 12, DT_F64 = 13,
};

__device__ __forceinline__ double load_any(const void *p, int64_t i, int dt) {
  switch (dt) {
    case DT_F32: return (double)((const float *)p)[i];
    case DT_F16: return (double)f16_to_f32(((const uint16_t *)p)[i]);
    case DT_BF16: return (double)bf16_to_f32(((const uint16_t *)p)[i]);
    case DT_E4M3: return (double)e4m3_to_f32(((const uint8_t *)p)[i]);
    case DT_I8: return (double)((const int8_t *)p)[i];
    case DT_I16: return (double)((const int16_t *)p)[i];
    case DT_I32: return (double)((const int32_t *)p)[i];
    case DT_I64: return (double)((const int64_t *)p)[i];
    case DT_U8: return (double)((const uint8_t *)p)[i];
    case DT_U16: return (double)((const uint16_t *)p)[i];
    case DT_U32: return (double)((const uint32_t *)p)[i];
    case DT_U64: return (double)((const uint64_t *)p)[i];
    case DT_BOOL: return ((const uint8_t *)p)[i] ? 1.0 : 0.0;
    case DT_F64: return ((const double *)p)[i];
  }
  return 0.0;
}

// E4M3FN encode, round to nearest even, saturating to +-448.
__device__ __forceinline__ uint8_t f32_to_e4m3(float f) {
  uint32_t u = __float_as_uint(f);
  uint8_t sign = (u >> 24) & 0x80;
  float a = fabsf(f);
  if (a != a) return 0x7f;
  if (a >= 448.f) return sign | 0x7e;
  if (a < 0.0009765625f) {  // below half the smallest subnormal (2^-10)
    return sign;
  }
  int e;
  float m = frexpf(a, &e);  // a = m * 2^e, m in [0.5, 1)
  int exp = e - 1 + 7;      // biased exponent of the 1.xxx form
  uint32_t code;
  if (exp <= 0) {
    // subnormal: value = k * 2^-9, k = 0..7
    float k = rintf(a * 512.f);
    code = (uint32_t)k;  // k == 8 rolls into the smallest normal (0x08)
  } else {
    float q = rintf((m * 2.f - 1.f) * 8.f);  // mantissa 0..8
    uint32_t mant = (uint32_t)q;
    if (mant == 8) { mant = 0; exp += 1; }
    code = ((uint32_t)exp << 3) | mant;
    if (code > 0x7e) code = 0x7e;
  }
  return sign | (uint8_t)code;
}

__device__ __forceinline__ double round_to_dtype(double v, int dt) {
  switch (dt) {
    case DT_F32: return (double)(float)v;
    case DT_F16: return (double)f16_to_f32(f32_to_f16((float)v));
    case DT_BF16: return (double)bf16_to_f32(f32_to_bf16((float)v));
    case DT_E4M3: return (double)e4m3_to_f32(f32_to_e4m3((float)v));
    case DT_I8: return (double)(int8_t)(int64_t)v;
    case DT_I16: return (double)(int16_t)(int64_t)v;
    case DT_I32: return (double)(int32_t)(int64_t)v;
    case DT_I64: return (double)(int64_t)v;
    case DT_U8: return (double)(uint8_t)(int64_t)v;
    case DT_U16: return (double)(uint16_t)(int64_t)v;
    case DT_U32: return (double)(uint32_t)(int64_t)v;
    case DT_U64: return (double)(uint64_t)v;
    case DT_BOOL: return v != 0.0 ? 1.0 : 0.0;
  }
  return v;
}

__device__ __forceinline__ void store_any(void *p, int64_t i, int dt, double v) {
  switch (dt) {
    case DT_F32: ((float *)p)[i] = (float)v; break;
    case DT_F16: ((uint16_t *)p)[i] = f32_to_f16((float)v); break;
    case DT_BF16: ((uint16_t *)p)[i] = f32_to_bf16((float)v); break;
    case DT_E4M3: ((uint8_t *)p)[i] = f32_to_e4m3((float)v); break;
    case DT_I8: ((int8_t *)p)[i] = (int8_t)(int64_t)v; break;
    case DT_I16: ((int16_t *)p)[i] = (int16_t)(int64_t)v; break;
    case DT_I32: ((int32_t *)p)[i] = (int32_t)(int64_t)v; break;
    case DT_I64: ((int64_t *)p)[i] = (int64_t)v; break;
    case DT_U8: ((uint8_t *)p)[i] = (uint8_t)(int64_t)v; break;
    case DT_U16: ((uint16_t *)p)[i] = (uint16_t)(int64_t)v; break;
    case DT_U32: ((uint32_t *)p)[i] = (uint32_t)(int64_t)v; break;
    case DT_U64: ((uint64_t *)p)[i] = (uint64_t)v; break;
    case DT_BOOL: ((uint8_t *)p)[i] = v != 0.0 ? 1 : 0; break;
    case DT_F64: ((double *)p)[i] = v; break;
  }
}

// ---------------------------------------------------------------------------
// Elementwise program
// ---------------------------------------------------------------------------
#define EW_MAX_RANK 6
#define EW_MAX_IN 8
#define EW_MAX_INSTR 40
#define EW_REGS 16

enum EwOp : int16_t {
  OP_LOAD = 0, OP_CONST, OP_IOTA,
  // unary
  OP_NEG = 10, OP_ABS, OP_EXP, OP_LOG, OP_SQRT, OP_RSQRT, OP_SIN, OP_COS, OP_TAN,
  OP_ATAN, OP_TANH, OP_CEIL, OP_FLOOR, OP_RINT, OP_TRUNC, OP_SIGN, OP_NOT, OP_LOG1P,
  OP_EXPM1, OP_ISFINITE, OP_ISNAN, OP_LOGISTIC, OP_LOG2, OP_COPY,
  // binary
  OP_ADD = 40, OP_SUB, OP_MUL, OP_DIV, OP_POW, OP_MAX, OP_MIN, OP_AND, OP_OR, OP_XOR,
  OP_REM, OP_FLOORDIV, OP_ATAN2,
  // compare
  OP_EQ = 60, OP_NE, OP_LT, OP_LE, OP_GT, OP_GE,
  // ternary
  OP_SELECT = 70,
};

struct EwInput {
  const void *ptr;
  int64_t strides[EW_MAX_RANK];  // in elements, over the output index space
  int32_t dtype;
  int32_t pad;
};

struct EwInstr {
  int16_t op;
  int8_t dst, a, b, c;
  int8_t dtype;  // result dtype (rounding) ; for OP_LOAD: unused
  int8_t flags;  // bit0: operands are integers (integer semantics)
  double imm;    // OP_CONST value; OP_IOTA dimension; OP_LOAD input index
};

struct EwArgs {
  void *out;
  int64_t out_offset;                // elements
  int64_t out_strides[EW_MAX_RANK];  // elements
  int64_t shape[EW_MAX_RANK];
  int64_t total;
  int32_t rank, n_in, n_instr, out_dtype;
  int32_t result_reg, pad;
  int64_t nthreads;  // grid size * 256 (grid-stride loop step)
  EwInput in[EW_MAX_IN];
  EwInstr prog[EW_MAX_INSTR];
};

__device__ __forceinline__ double floor_mod(double a, double b, bool isint) {
  if (isint) {
    int64_t x = (int64_t)a, y = (int64_t)b;
    if (y == 0) return 0.0;
    int64_t r = x % y;
    if (r != 0 && ((r < 0) != (y < 0))) r += y;
    return (double)r;
  }
  double r = fmod(a, b);
  if (r != 0.0 && ((r < 0.0) != (b < 0.0))) r += b;
  return r;
}

__device__ __forceinline__ double floor_div(double a, double b, bool isint) {
  if (isint) {
    int64_t x = (int64_t)a, y = (int64_t)b;
    if (y == 0) return 0.0;
    int64_t q = x / y;
    if ((x % y != 0) && ((x < 0) != (y < 0))) q -= 1;
    return (double)q;
  }
  return floor(a / b);
}

extern "C" __global__ __launch_bounds__(256) void nk_ew_program(EwArgs a) {
  const int64_t stride = a.nthreads;
  for (int64_t lin = (int64_t)blockIdx.x * 256 + threadIdx.x; lin < a.total; lin += stride) {
    int64_t idx[EW_MAX_RANK];
    int64_t rem = lin;
    for (int d = a.rank - 1; d >= 0; --d) {
      idx[d] = rem % a.shape[d];
      rem /= a.shape[d];
    }
    double r[EW_REGS];
    for (int k = 0; k < a.n_instr; ++k) {
      const EwInstr &I = a.prog[k];
      const bool isint = I.flags & 1;
      double x = r[I.a & (EW_REGS - 1)];
      double y = r[I.b & (EW_REGS - 1)];
      double v = 0.0;
      switch (I.op) {
        case OP_LOAD: {
          const EwInput &in = a.in[(int)I.imm];
          int64_t off = 0;
          for (int d = 0; d < a.rank; ++d) off += idx[d] * in.strides[d];
          v = load_any(in.ptr, off, in.dtype);
          break;
        }
        case OP_CONST: v = I.imm; break;
        case OP_IOTA: v = (double)idx[(int)I.imm]; break;
        case OP_NEG: v = -x; break;
        case OP_ABS: v = fabs(x); break;
        case OP_EXP: v = exp(x); break;
        case OP_LOG: v = log(x); break;
        case OP_SQRT: v = sqrt(x); break;
        case OP_RSQRT: v = 1.0 / sqrt(x); break;
        case OP_SIN: v = sin(x); break;
        case OP_COS: v = cos(x); break;
        case OP_TAN: v = tan(x); break;
        case OP_ATAN: v = atan(x); break;
        case OP_TANH: v = tanh(x); break;
        case OP_CEIL: v = ceil(x); break;
        case OP_FLOOR: v = floor(x); break;
        case OP_RINT: v = rint(x); break;
        case OP_TRUNC: v = trunc(x); break;
        case OP_SIGN: v = (x > 0.0) ? 1.0 : ((x < 0.0) ? -1.0 : x); break;
        case OP_NOT: v = (I.dtype == DT_BOOL) ? (x != 0.0 ? 0.0 : 1.0) : (double)(~(int64_t)x); break;
        case OP_LOG1P: v = log1p(x); break;
        case OP_EXPM1: v = expm1(x); break;
        case OP_ISFINITE: v = isfinite(x) ? 1.0 : 0.0; break;
        case OP_ISNAN: v = isnan(x) ? 1.0 : 0.0; break;
        case OP_LOGISTIC: v = 1.0 / (1.0 + exp(-x)); break;
        case OP_LOG2: v = log2(x); break;
        case OP_COPY: v = x; break;
        case OP_ADD: v = x + y; break;
        case OP_SUB: v = x - y; break;
        case OP_MUL: v = x * y; break;
        case OP_DIV:
          if (isint) v = (y == 0.0) ? 0.0 : (double)((int64_t)x / (int64_t)y);
          else v = x / y;
          break;
        case OP_POW: v = pow(x, y); break;
        case OP_MAX: v = (x != x || y != y) ? (x + y) : fmax(x, y); break;
        case OP_MIN: v = (x != x || y != y) ? (x + y) : fmin(x, y); break;
        case OP_AND: v = (double)((int64_t)x & (int64_t)y); break;
        case OP_OR: v = (double)((int64_t)x | (int64_t)y); break;
        case OP_XOR: v = (double)((int64_t)x ^ (int64_t)y); break;
        case OP_REM: v = floor_mod(x, y, isint); break;
        case OP_FLOORDIV: v = floor_div(x, y, isint); break;
        case OP_ATAN2: v = atan2(x, y); break;
        case OP_EQ: v = x == y; break;
        case OP_NE: v = x != y; break;
        case OP_LT: v = x < y; break;
        case OP_LE: v = x <= y; break;
        case OP_GT: v = x > y; break;
        case OP_GE: v = x >= y; break;
        case OP_SELECT: v = (x != 0.0) ? y : r[I.c & (EW_REGS - 1)]; break;
      }
      r[I.dst & (EW_REGS - 1)] = round_to_dtype(v, I.dtype);
    }
    int64_t off = a.out_offset;
    for (int d = 0; d < a.rank; ++d) off += idx[d] * a.out_strides[d];
    store_any(a.out, off, a.out_dtype, r[a.result_reg & (EW_REGS - 1)]);
  }
}

// ---------------------------------------------------------------------------
// Reduction: one workgroup per output element.
// ---------------------------------------------------------------------------
#define RED_MAX_RANK 6
enum RedOp : int32_t { RED_ADD = 0, RED_MAX, RED_MIN, RED_MUL, RED_AND, RED_OR, RED_ARGMAX, RED_ARGMIN };

struct ReduceArgs {
  const void *in;
  void *out;
  int64_t out_shape[RED_MAX_RANK];
  int64_t out_strides[RED_MAX_RANK];  // input strides of the kept axes
  int64_t red_shape[RED_MAX_RANK];
  int64_t red_strides[RED_MAX_RANK];  // input strides of the reduced axes
  int64_t n_out, n_red;
  int32_t out_rank, red_rank, op, in_dtype, out_dtype, acc_f32;
};

__device__ __forceinline__ double red_init(int op) {
  switch (op) {
    case RED_ADD: case RED_OR: return 0.0;
    case RED_MUL: case RED_AND: return 1.0;
    case RED_MAX: case RED_ARGMAX: return -INFINITY;
    default: return INFINITY;
  }
}

__device__ __forceinline__ double red_comb(int op, double a, double b) {
  switch (op) {
    case RED_ADD: return a + b;
    case RED_MUL: return a * b;
    case RED_MAX: return (a != a || b != b) ? a + b : fmax(a, b);
    case RED_MIN: return (a != a || b != b) ? a + b : fmin(a, b);
    case RED_AND: return (a != 0.0 && b != 0.0) ? 1.0 : 0.0;
    case RED_OR: return (a != 0.0 || b != 0.0) ? 1.0 : 0.0;
  }
  return a;
}

extern "C" __global__ __launch_bounds__(256) void nk_reduce(ReduceArgs a) {
  __shared__ double sv[256];
  __shared__ int64_t si[256];
  const int64_t o = blockIdx.x;
  if (o >= a.n_out) return;
  int64_t base = 0, rem = o;
  for (int d = a.out_rank - 1; d >= 0; --d) {
    base += (rem % a.out_shape[d]) * a.out_strides[d];
    rem /= a.out_shape[d];
  }
  const bool arg = a.op == RED_ARGMAX || a.op == RED_ARGMIN;
  const bool amax = a.op == RED_ARGMAX;
  double acc = red_init(a.op);
  int64_t best = a.n_red;  // sentinel: no element seen
  for (int64_t j = threadIdx.x; j < a.n_red; j += 256) {
    int64_t off = base, r2 = j;
    for (int d = a.red_rank - 1; d >= 0; --d) {
      off += (r2 % a.red_shape[d]) * a.red_strides[d];
      r2 /= a.red_shape[d];
    }
    double v = load_any(a.in, off, a.in_dtype);
    if (arg) {
      // first occurrence wins; a NaN beats any number (NumPy semantics)
      bool take = best == a.n_red ||
                  (acc == acc && (v != v || (amax ? v > acc : v < acc)));
      if (take) { acc = v; best = j; }
    } else {
      acc = red_comb(a.op, acc, v);
      if (a.acc_f32) acc = (double)(float)acc;
    }
  }
  sv[threadIdx.x] = acc;
  si[threadIdx.x] = best;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) {
      double x = sv[threadIdx.x], y = sv[threadIdx.x + s];
      if (arg) {
        int64_t ix = si[threadIdx.x], iy = si[threadIdx.x + s];
        bool take_y = false;
        if (iy < a.n_red) {
          if (ix >= a.n_red) take_y = true;
          else if (x != x) take_y = (y != y) && iy < ix;
          else if (y != y) take_y = true;
          else if (amax ? y > x : y < x) take_y = true;
          else if (y == x && iy < ix) take_y = true;
        }
        if (take_y) { sv[threadIdx.x] = y; si[threadIdx.x] = iy; }
      } else {
        double z = red_comb(a.op, x, y);
        sv[threadIdx.x] = a.acc_f32 ? (double)(float)z : z;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (arg) store_any(a.out, o, a.out_dtype, (double)si[0]);
    else store_any(a.out, o, a.out_dtype, sv[0]);
  }
}

// ---------------------------------------------------------------------------
// Generic batched dot: C[b, m, n] = sum_k A[b, m, k] * B[b, k, n]
// ---------------------------------------------------------------------------
struct DotArgs {
  const void *A;
  const void *B;
  void *C;
  int64_t batch, M, N, K;
  int64_t sab, sam, sak;  // A strides (elements)
  int64_t sbb, sbk, sbn;  // B strides
  int32_t a_dtype, b_dtype, c_dtype, pad;
};

#define DT_TILE 16
extern "C" __global__ __launch_bounds__(256) void nk_dot(DotArgs a) {
  __shared__ float As[DT_TILE][DT_TILE + 1];
  __shared__ float Bs[DT_TILE][DT_TILE + 1];
  const int64_t b = blockIdx.z;
  const int tx = threadIdx.x % DT_TILE, ty = threadIdx.x / DT_TILE;
  const int64_t m = (int64_t)blockIdx.y * DT_TILE + ty;
  const int64_t n = (int64_t)blockIdx.x * DT_TILE + tx;
  float acc = 0.f;
  for (int64_t k0 = 0; k0 < a.K; k0 += DT_TILE) {
    int64_t ka = k0 + tx, kb = k0 + ty;
    As[ty][tx] = (m < a.M && ka < a.K) ? (float)load_any(a.A, b * a.sab + m * a.sam + ka * a.sak, a.a_dtype) : 0.f;
    Bs[ty][tx] = (kb < a.K && n < a.N) ? (float)load_any(a.B, b * a.sbb + kb * a.sbk + n * a.sbn, a.b_dtype) : 0.f;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < DT_TILE; ++k) acc = fmaf(As[ty][k], Bs[k][tx], acc);
    __syncthreads();
  }
  if (m < a.M && n < a.N) store_any(a.C, (b * a.M + m) * a.N + n, a.c_dtype, (double)acc);
}

// ---------------------------------------------------------------------------
// Gather / scatter along one axis.  Operands are viewed as (O, A, N):
// O = product of the axes before `axis`, A = the axis, N = the axes after.
//   mode 0 take:            out[o, i, n] = in[o, idx[i], n]           (I = #idx)
//   mode 1 take_along_axis: out[o, i, n] = in[o, idx[o, i, n], n]
//   mode 2 scatter:         out[o, idx[i], n] = upd[o, i, n]
//   mode 3 put_along_axis:  out[o, idx[o, i, n], n] = upd[o, i, n]
// Modes 2/3 expect `out` to already hold the operand.
// ---------------------------------------------------------------------------
struct GatherArgs {
  const void *src;  // in (modes 0/1) or updates (modes 2/3)
  const int32_t *idx;
  void *out;
  int64_t O, A, I, N;
  int64_t nthreads;  // grid size * 256
  int32_t mode, dtype;
};

extern "C" __global__ __launch_bounds__(256) void nk_gather(GatherArgs a) {
  const int64_t total = a.O * a.I * a.N;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += a.nthreads) {
    const int64_t n = t % a.N;
    const int64_t i = (t / a.N) % a.I;
    const int64_t o = t / (a.N * a.I);
    int64_t j = (a.mode == 0 || a.mode == 2) ? a.idx[i] : a.idx[t];
    if (j < 0) j += a.A;
    const bool ok = j >= 0 && j < a.A;
    if (a.mode <= 1) {
      j = j < 0 ? 0 : (j >= a.A ? a.A - 1 : j);
      store_any(a.out, t, a.dtype, load_any(a.src, (o * a.A + j) * a.N + n, a.dtype));
    } else if (ok) {
      store_any(a.out, (o * a.A + j) * a.N + n, a.dtype, load_any(a.src, t, a.dtype));
    }
  }
}

// ---------------------------------------------------------------------------
// Inclusive cumulative sum along an axis viewed as (O, A, N).
// ---------------------------------------------------------------------------
struct CumsumArgs {
  const void *in;
  void *out;
  int64_t O, A, N;
  int32_t in_dtype, out_dtype, acc_f32, pad;
};

extern "C" __global__ __launch_bounds__(256) void nk_cumsum(CumsumArgs a) {
  const int64_t line = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (line >= a.O * a.N) return;
  const int64_t o = line / a.N, n = line % a.N;
  double acc = 0.0;
  for (int64_t i = 0; i < a.A; ++i) {
    const int64_t off = (o * a.A + i) * a.N + n;
    acc += load_any(a.in, off, a.in_dtype);
    if (a.acc_f32) acc = (double)(float)acc;
    store_any(a.out, off, a.out_dtype, acc);
  }
}

// ---------------------------------------------------------------------------
// Streaming copy of n16 16-byte words (plan flat copies; also the plain copy
// kernel of known size that calibrates the HBM traffic counters).
// ---------------------------------------------------------------------------
struct Copy16Args {
  const uint4 *src;
  uint4 *dst;
  int64_t n16;
  int64_t nthreads;  // grid size * 256
};

extern "C" __global__ __launch_bounds__(256) void nk_copy16(Copy16Args a) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < a.n16; i += a.nthreads)
    nt_store16(a.dst + i, nt_load16(a.src + i));
}

// fp8 E4M3FN codes -> bf16 with the decode the GEMM staging uses (8 codes per
// thread).  Weight preparation and the exhaustive check of the decode.
struct DecodeE4m3Args {
  const uint2 *src;
  uint4 *dst;
  int64_t n8;
  int64_t nthreads;
};

extern "C" __global__ __launch_bounds__(256) void nk_decode_e4m3_bf16(DecodeE4m3Args a) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < a.n8; i += a.nthreads)
    a.dst[i] = e4m3x8_to_bf16x8(a.src[i]);
}

// Row-wise top-k (indices) along the last axis: one workgroup per row.
// Round r selects, among the elements that come after round r-1's pick in
// the order (value descending, index ascending) -- ascending values when
// `largest` is 0 -- the first one; each round is one pass over the row, so
// the input is never modified.  k is small (sampling); rows must not hold
// NaN.
struct TopkArgs {
  const void *in;
  uint32_t *idx;  // rows x k
  int64_t rows;
  int64_t n;
  int32_t k;
  int32_t largest;
  int32_t dtype;
  int32_t pad;
};

extern "C" __global__ __launch_bounds__(256) void nk_topk(TopkArgs a) {
  __shared__ double sv[256];
  __shared__ int64_t si[256];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t base = row * a.n;
  const double sgn = a.largest ? 1.0 : -1.0;
  double pv = 0.0;
  int64_t pi = -1;  // previous pick (none before round 0)
  for (int r = 0; r < a.k; ++r) {
    double bv = -INFINITY;
    int64_t bi = a.n;
    for (int64_t j = tid; j < a.n; j += 256) {
      const double v = sgn * load_any(a.in, base + j, a.dtype);
      const bool after = pi < 0 || v < pv || (v == pv && j > pi);
      if (after && (v > bv || (v == bv && j < bi))) {
        bv = v;
        bi = j;
      }
    }
    sv[tid] = bv;
    si[tid] = bi;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
      if (tid < s) {
        const double ov = sv[tid + s];
        const int64_t oi = si[tid + s];
        if (ov > sv[tid] || (ov == sv[tid] && oi < si[tid])) {
          sv[tid] = ov;
          si[tid] = oi;
        }
      }
      __syncthreads();
    }
    pv = sv[0];
    pi = si[0] < a.n ? si[0] : a.n - 1;  // a row shorter than k repeats its last pick
    if (tid == 0) a.idx[row * a.k + r] = (uint32_t)pi;
    __syncthreads();
  }
}
