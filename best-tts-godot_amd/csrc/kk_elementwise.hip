// Broadcast elementwise family, strided copy/cast, fill and gather.
//
// One engine serves every elementwise node: the host plans the launch
// (broadcast strides, unit-axis removal, contiguous-axis merging) and picks
//  * fast paths, all operands fp32 with the collapsed innermost axis
//    contiguous (stride 1) or broadcast (stride 0) for every operand; each
//    thread owns VEC consecutive elements of a row (128-bit non-temporal
//    loads and stores when VEC == 4):
//      ew_rows<OP, NIN, VEC>      rank <= 2, rows on blockIdx.y.  The hot
//                                 shapes land here: x [1,C,L] op [1,C,1]
//                                 collapses to [C, L] with strides (L,1) and
//                                 (1,0), so the per-channel value is one
//                                 block-uniform load.
//      ew_inner<OP, NIN, VEC, Idx> rank > 2, outer offsets from a div/mod
//                                 walk once per VEC elements.
//  * ew_generic: any dtype mix, any strides, one element per thread.
// All walk grid-stride loops so any size fits any grid.
#include <algorithm>

#include "kk_internal.h"

namespace kk {

// Composite ops that only exist inside the library.
enum {
  OPX_SNAKE = 100,        // a=x, b=alpha, c=recip
  OPX_SNAKE_ALPHA = 101,  // a=x, b=alpha, recip = 1/alpha
  OPX_FASTGELU = 102,     // a=x, b=bias (0 if absent)
  OPX_DEQUANT = 103,      // a=q, b=scale, c=zp
  OPX_CLIP = 104,         // a=x, b=lo, c=hi (flags in `aux`)
  OPX_WHERE = 105,        // a=cond, b=x, c=y
  OPX_COPY = 106,         // a -> out with dtype conversion
  OPX_FASTGELU_NB = 107   // a=x, no bias
};

constexpr int kMaxArgRank = KK_MAX_RANK;

struct EwArgs {
  int rank;
  int op;
  float alpha;
  int aux;
  int dt[kMaxOperands];        // 0 = out
  const void* in[kMaxOperands - 1];
  void* out;
  int64_t n;
  int64_t dims[kMaxArgRank];
  int64_t st[kMaxOperands][kMaxArgRank];
};

// numpy's minimum/maximum propagate NaN from either side.
__device__ __forceinline__ float np_min(float a, float b) {
  if (__builtin_isnan(a) || __builtin_isnan(b)) return a + b;
  return a < b ? a : b;
}
__device__ __forceinline__ float np_max(float a, float b) {
  if (__builtin_isnan(a) || __builtin_isnan(b)) return a + b;
  return a > b ? a : b;
}

// fp32 semantics of each op, written in the evaluation order of the numpy
// expression it mirrors (tools/ref_runtime.py:446-489, :288-293) so that
// correctly rounded ops (+ - * / sqrt) give identical bits.  The library is
// built with -ffp-contract=off: no FMA is formed behind our back.
template <int OP>
__device__ __forceinline__ float apply_f32(float a, float b, float c, float alpha, int aux) {
  if constexpr (OP == KK_OP_ADD) return a + b;
  else if constexpr (OP == KK_OP_SUB) return a - b;
  else if constexpr (OP == KK_OP_MUL) return a * b;
  else if constexpr (OP == KK_OP_DIV) return a / b;
  else if constexpr (OP == KK_OP_POW) return b == 2.0f ? a * a : powf(a, b);
  else if constexpr (OP == KK_OP_SQRT) return sqrtf(a);
  else if constexpr (OP == KK_OP_EXP) return expf(a);
  else if constexpr (OP == KK_OP_SIN) return kk_sin(a);
  else if constexpr (OP == KK_OP_COS) return cosf(a);
  else if constexpr (OP == KK_OP_ATAN) return atanf(a);
  else if constexpr (OP == KK_OP_TANH) return tanhf(a);
  else if constexpr (OP == KK_OP_SIGMOID) return 1.0f / (1.0f + expf(-a));
  else if constexpr (OP == KK_OP_FLOOR) return floorf(a);
  else if constexpr (OP == KK_OP_ROUND) return rintf(a);
  else if constexpr (OP == KK_OP_LEAKYRELU) return a < 0.0f ? a * alpha : a;
  else if constexpr (OP == KK_OP_NEG) return -a;
  else if constexpr (OP == KK_OP_ABS) return fabsf(a);
  else if constexpr (OP == KK_OP_LOG) return logf(a);
  else if constexpr (OP == KK_OP_ERF) return erff(a);
  else if constexpr (OP == KK_OP_MIN) return np_min(a, b);
  else if constexpr (OP == KK_OP_MAX) return np_max(a, b);
  else if constexpr (OP == KK_OP_IDENTITY || OP == OPX_COPY) return a;
  else if constexpr (OP == OPX_SNAKE || OP == OPX_SNAKE_ALPHA) {
    // Mul(alpha, x) -> Sin -> Pow(., 2) -> Mul(recip, .) -> Add(x, .)
    const float r = (OP == OPX_SNAKE) ? c : 1.0f / b;
    const float p = kk_sin_sq(b * a);
    const float q = r * p;
    return a + q;
  } else if constexpr (OP == OPX_FASTGELU || OP == OPX_FASTGELU_NB) {
    // op_fast_gelu: x += bias; 0.5*x*(1 + tanh(c*(x + 0.044715*x*x*x)))
    const float x = (OP == OPX_FASTGELU) ? a + b : a;
    float t = 0.044715f * x;
    t = t * x;
    t = t * x;
    t = x + t;
    t = 0.7978845608028654f * t;
    const float th = tanhf(t);
    return (0.5f * x) * (1.0f + th);
  } else if constexpr (OP == OPX_DEQUANT) {
    return (a - c) * b;
  } else if constexpr (OP == OPX_CLIP) {
    float v = a;
    if (aux & 1) v = np_max(v, b);
    if (aux & 2) v = np_min(v, c);
    return v;
  } else {
    return a;
  }
}

// Row offset of operand k for collapsed row index `row` over the outer axes
// [0, rank-1).
template <typename Idx>
__device__ __forceinline__ void outer_offsets(const EwArgs& A, Idx row, Idx (&off)[kMaxOperands],
                                              int nops) {
#pragma unroll
  for (int k = 0; k < kMaxOperands; ++k) off[k] = 0;
  for (int d = A.rank - 2; d >= 0; --d) {
    const Idx sz = static_cast<Idx>(A.dims[d]);
    const Idx coord = row % sz;
    row /= sz;
#pragma unroll
    for (int k = 0; k < kMaxOperands; ++k)
      if (k < nops) off[k] += coord * static_cast<Idx>(A.st[k][d]);
  }
}

// Loads VEC consecutive floats of an operand whose innermost stride is 1
// (streamed) or 0 (one value broadcast along the row).
template <int VEC>
__device__ __forceinline__ void load_operand(const float* __restrict__ p, bool contiguous,
                                             float (&v)[VEC]) {
  if constexpr (VEC == 4) {
    if (contiguous) {
      const float4 t = ld_stream4(p);
      v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    } else {
      v[0] = v[1] = v[2] = v[3] = *p;
    }
  } else {
    v[0] = contiguous ? ld_stream(p) : *p;
  }
}

template <int OP, int NIN, int VEC>
__device__ __forceinline__ void ew_apply_store(float* __restrict__ out, const float (&a)[VEC],
                                               const float (&b)[VEC], const float (&c)[VEC],
                                               float alpha, int aux) {
  float r[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i)
    r[i] = apply_f32<OP>(a[i], NIN > 1 ? b[i] : 0.0f, NIN > 2 ? c[i] : 0.0f, alpha, aux);
  if constexpr (VEC == 4) st_stream4(out, make_float4(r[0], r[1], r[2], r[3]));
  else st_stream(out, r[0]);
}

// Plans of rank <= 2: [rows, L].  Rows run over blockIdx.y, so each operand's
// row offset -- and a row-broadcast operand's value -- is uniform across the
// block; columns run over blockIdx.x with one VEC-wide item per thread.
template <int OP, int NIN, int VEC>
__global__ void __launch_bounds__(256) ew_rows(EwArgs A) {
  const int64_t L = A.dims[A.rank - 1];
  const int64_t rows = A.rank == 2 ? A.dims[0] : 1;
  const int64_t per_row = L / VEC;
  float* __restrict__ out = static_cast<float*>(A.out);
  const float* __restrict__ in0 = static_cast<const float*>(A.in[0]);
  const float* __restrict__ in1 = NIN > 1 ? static_cast<const float*>(A.in[1]) : nullptr;
  const float* __restrict__ in2 = NIN > 2 ? static_cast<const float*>(A.in[2]) : nullptr;
  const int last = A.rank - 1;
  const bool c0 = A.st[1][last] != 0, c1 = NIN > 1 && A.st[2][last] != 0,
             c2 = NIN > 2 && A.st[3][last] != 0;
  for (int64_t row = blockIdx.y; row < rows; row += gridDim.y) {
    const int64_t ro = A.rank == 2 ? row * A.st[0][0] : 0;
    const int64_t r0 = A.rank == 2 ? row * A.st[1][0] : 0;
    const int64_t r1 = (NIN > 1 && A.rank == 2) ? row * A.st[2][0] : 0;
    const int64_t r2 = (NIN > 2 && A.rank == 2) ? row * A.st[3][0] : 0;
    for (int64_t v = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; v < per_row;
         v += static_cast<int64_t>(gridDim.x) * blockDim.x) {
      const int64_t col = v * VEC;
      float a[VEC], b[VEC], c[VEC];
      load_operand<VEC>(in0 + r0 + (c0 ? col : 0), c0, a);
      if constexpr (NIN > 1) load_operand<VEC>(in1 + r1 + (c1 ? col : 0), c1, b);
      if constexpr (NIN > 2) load_operand<VEC>(in2 + r2 + (c2 ? col : 0), c2, c);
      ew_apply_store<OP, NIN, VEC>(out + ro + col, a, b, c, A.alpha, A.aux);
    }
  }
}

// Plans of rank <= 2 whose rows are not whole float4s (L % 4 != 0, L >= 4)
// but whose output is contiguous: the output is walked flat, four elements
// at a time.  Each input is flat (contiguous like the output: one float4
// load), per-row (one value per row, the item's row and, where the item
// runs past the row's end, the next one) or a scalar; `kinds` holds two
// bits per input (0 flat, 1 per-row).
template <int OP, int NIN>
__global__ void __launch_bounds__(256) ew_flat4(EwArgs A, int kinds) {
  const int64_t L = A.dims[A.rank - 1];
  const int64_t n = A.n;
  const double invL = 1.0 / static_cast<double>(L);
  float* __restrict__ out = static_cast<float*>(A.out);
  const float* __restrict__ in[3] = {static_cast<const float*>(A.in[0]),
                                     NIN > 1 ? static_cast<const float*>(A.in[1]) : nullptr,
                                     NIN > 2 ? static_cast<const float*>(A.in[2]) : nullptr};
  const int64_t rst[3] = {A.rank == 2 ? A.st[1][0] : 0, A.rank == 2 ? A.st[2][0] : 0,
                          A.rank == 2 ? A.st[3][0] : 0};
  auto locate = [&](int64_t i, int64_t& row, int64_t& col) {
    row = static_cast<int64_t>(static_cast<double>(i) * invL);
    col = i - row * L;
    if (col < 0) { --row; col += L; } else if (col >= L) { ++row; col -= L; }
  };
  const int64_t items = n / 4;
  for (int64_t v = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; v < items;
       v += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i = 4 * v;
    int64_t row, col;
    locate(i, row, col);
    float x[3][4];
#pragma unroll
    for (int k = 0; k < NIN; ++k) {
      if (((kinds >> (2 * k)) & 3) == 0) {
        const float4 t = ld_stream4(in[k] + i);
        x[k][0] = t.x; x[k][1] = t.y; x[k][2] = t.z; x[k][3] = t.w;
      } else {
        const float r0 = in[k][row * rst[k]];
        const float r1 = col + 3 >= L ? in[k][(row + 1) * rst[k]] : r0;
#pragma unroll
        for (int e = 0; e < 4; ++e) x[k][e] = col + e < L ? r0 : r1;
      }
    }
    float r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      r[e] = apply_f32<OP>(x[0][e], NIN > 1 ? x[1][e] : 0.0f, NIN > 2 ? x[2][e] : 0.0f, A.alpha,
                           A.aux);
    st_stream4(out + i, make_float4(r[0], r[1], r[2], r[3]));
  }
  // the last n % 4 elements
  if (blockIdx.x == 0 && threadIdx.x < n - 4 * items) {
    const int64_t i = 4 * items + threadIdx.x;
    int64_t row, col;
    locate(i, row, col);
    float x[3];
#pragma unroll
    for (int k = 0; k < NIN; ++k)
      x[k] = ((kinds >> (2 * k)) & 3) == 0 ? in[k][i] : in[k][row * rst[k]];
    out[i] = apply_f32<OP>(x[0], NIN > 1 ? x[1] : 0.0f, NIN > 2 ? x[2] : 0.0f, A.alpha, A.aux);
  }
}

// Plans of rank > 2: flat index over VEC-wide items; the outer offsets come
// from a div/mod walk over the outer axes.
template <int OP, int NIN, int VEC, typename Idx>
__global__ void __launch_bounds__(256) ew_inner(EwArgs A) {
  const Idx L = static_cast<Idx>(A.dims[A.rank - 1]);
  const Idx per_row = L / VEC;
  const Idx items = static_cast<Idx>(A.n) / VEC;
  float* __restrict__ out = static_cast<float*>(A.out);
  const float* __restrict__ in0 = static_cast<const float*>(A.in[0]);
  const float* __restrict__ in1 = NIN > 1 ? static_cast<const float*>(A.in[1]) : nullptr;
  const float* __restrict__ in2 = NIN > 2 ? static_cast<const float*>(A.in[2]) : nullptr;
  const bool c0 = A.st[1][A.rank - 1] != 0;
  const bool c1 = NIN > 1 && A.st[2][A.rank - 1] != 0;
  const bool c2 = NIN > 2 && A.st[3][A.rank - 1] != 0;
  for (Idx v = blockIdx.x * static_cast<Idx>(blockDim.x) + threadIdx.x; v < items;
       v += static_cast<Idx>(gridDim.x) * blockDim.x) {
    const Idx row = v / per_row;
    const Idx col = (v - row * per_row) * VEC;
    Idx off[kMaxOperands];
    outer_offsets<Idx>(A, row, off, NIN + 1);
    float a[VEC], b[VEC], c[VEC];
    load_operand<VEC>(in0 + off[1] + (c0 ? col : 0), c0, a);
    if constexpr (NIN > 1) load_operand<VEC>(in1 + off[2] + (c1 ? col : 0), c1, b);
    if constexpr (NIN > 2) load_operand<VEC>(in2 + off[3] + (c2 ? col : 0), c2, c);
    ew_apply_store<OP, NIN, VEC>(out + off[0] + col, a, b, c, A.alpha, A.aux);
  }
}

// ----------------------------------------------------------- generic path
enum { MODE_FLOAT = 0, MODE_INT = 1, MODE_DOUBLE = 2 };

__device__ __forceinline__ void store_value(void* p, int dt, int64_t i, float fv, int64_t iv,
                                            bool is_f) {
  switch (dt) {
    case KK_F32: static_cast<float*>(p)[i] = is_f ? fv : static_cast<float>(iv); break;
    case KK_F16: static_cast<__half*>(p)[i] = __float2half(is_f ? fv : static_cast<float>(iv)); break;
    case KK_BOOL: static_cast<uint8_t*>(p)[i] = is_f ? (fv != 0.0f) : (iv != 0); break;
    default: {
      int64_t v = iv;
      if (is_f) {
        // float -> int truncates toward zero (numpy astype); NaN and values
        // beyond the int64 range give INT64_MIN like the x86 conversion.
        const float t = truncf(fv);
        v = (t >= -9.223372036854775808e18f && t < 9.223372036854775808e18f)
                ? static_cast<int64_t>(t) : INT64_MIN;
      }
      switch (dt) {
        case KK_I8: static_cast<int8_t*>(p)[i] = static_cast<int8_t>(v); break;
        case KK_U8: static_cast<uint8_t*>(p)[i] = static_cast<uint8_t>(v); break;
        case KK_I32: static_cast<int32_t*>(p)[i] = static_cast<int32_t>(v); break;
        case KK_I64: static_cast<int64_t*>(p)[i] = v; break;
      }
    }
  }
}

__device__ __forceinline__ float apply_runtime_f32(int op, float a, float b, float c, float alpha,
                                                   int aux) {
  switch (op) {
#define KK_CASE(OPC) case OPC: return apply_f32<OPC>(a, b, c, alpha, aux);
    KK_CASE(KK_OP_ADD) KK_CASE(KK_OP_SUB) KK_CASE(KK_OP_MUL) KK_CASE(KK_OP_DIV)
    KK_CASE(KK_OP_POW) KK_CASE(KK_OP_SQRT) KK_CASE(KK_OP_EXP) KK_CASE(KK_OP_SIN)
    KK_CASE(KK_OP_COS) KK_CASE(KK_OP_ATAN) KK_CASE(KK_OP_TANH) KK_CASE(KK_OP_SIGMOID)
    KK_CASE(KK_OP_FLOOR) KK_CASE(KK_OP_ROUND) KK_CASE(KK_OP_LEAKYRELU) KK_CASE(KK_OP_NEG)
    KK_CASE(KK_OP_ABS) KK_CASE(KK_OP_LOG) KK_CASE(KK_OP_ERF) KK_CASE(KK_OP_MIN)
    KK_CASE(KK_OP_MAX) KK_CASE(KK_OP_IDENTITY) KK_CASE(OPX_COPY) KK_CASE(OPX_SNAKE)
    KK_CASE(OPX_SNAKE_ALPHA) KK_CASE(OPX_FASTGELU) KK_CASE(OPX_FASTGELU_NB)
    KK_CASE(OPX_DEQUANT) KK_CASE(OPX_CLIP)
#undef KK_CASE
  }
  return a;
}

__device__ __forceinline__ int64_t floor_div(int64_t a, int64_t b) {
  if (b == 0) return 0;  // numpy returns 0 (with a warning) for x // 0
  int64_t q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
  return q;
}

__device__ __forceinline__ int64_t apply_i64(int op, int64_t a, int64_t b) {
  switch (op) {
    case KK_OP_ADD: return static_cast<int64_t>(static_cast<uint64_t>(a) + static_cast<uint64_t>(b));
    case KK_OP_SUB: return static_cast<int64_t>(static_cast<uint64_t>(a) - static_cast<uint64_t>(b));
    case KK_OP_MUL: return static_cast<int64_t>(static_cast<uint64_t>(a) * static_cast<uint64_t>(b));
    case KK_OP_DIV: return floor_div(a, b);
    case KK_OP_MIN: return a < b ? a : b;
    case KK_OP_MAX: return a > b ? a : b;
    case KK_OP_NEG: return -a;
    case KK_OP_ABS: return a < 0 ? -a : a;
    case KK_OP_IDENTITY: case OPX_COPY: return a;
  }
  return a;
}

__device__ __forceinline__ bool compare_op(int op, double a, double b) {
  switch (op) {
    case KK_OP_EQUAL: return a == b;
    case KK_OP_GREATER: return a > b;
    case KK_OP_LESS: return a < b;
    case KK_OP_GEQ: return a >= b;
    case KK_OP_AND: return (a != 0.0) && (b != 0.0);
  }
  return false;
}

__device__ __forceinline__ double load_as_f64(const void* p, int dt, int64_t i) {
  if (dt == KK_F32) return static_cast<const float*>(p)[i];
  if (dt == KK_F16) return __half2float(static_cast<const __half*>(p)[i]);
  return static_cast<double>(load_as_i64(p, dt, i));
}

__device__ __forceinline__ bool is_int_dt(int dt) { return !(dt == KK_F32 || dt == KK_F16); }

// `mode` selects the compute domain: fp32 (MODE_FLOAT), int64 (MODE_INT)
// or, for comparisons, exact double.
__global__ void __launch_bounds__(256) ew_generic(EwArgs A, int nin, int mode) {
  const int64_t n = A.n;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t rem = i;
    int64_t off[kMaxOperands] = {0, 0, 0, 0};
    for (int d = A.rank - 1; d >= 0; --d) {
      const int64_t sz = A.dims[d];
      const int64_t coord = rem % sz;
      rem /= sz;
#pragma unroll
      for (int k = 0; k < kMaxOperands; ++k) off[k] += coord * A.st[k][d];
    }
    const int op = A.op;
    if (op >= KK_OP_EQUAL && op <= KK_OP_AND) {
      const double a = load_as_f64(A.in[0], A.dt[1], off[1]);
      const double b = load_as_f64(A.in[1], A.dt[2], off[2]);
      store_value(A.out, A.dt[0], off[0], 0.0f, compare_op(op, a, b) ? 1 : 0, false);
    } else if (op == OPX_WHERE) {
      const bool cnd = load_as_f64(A.in[0], A.dt[1], off[1]) != 0.0;
      const int src = cnd ? 1 : 2;
      const void* p = A.in[src];
      const int dt = A.dt[src + 1];
      if (mode == MODE_INT)
        store_value(A.out, A.dt[0], off[0], 0.0f, load_as_i64(p, dt, off[src + 1]), false);
      else
        store_value(A.out, A.dt[0], off[0], load_as_f32(p, dt, off[src + 1]), 0, true);
    } else if (mode == MODE_INT) {
      const int64_t a = load_as_i64(A.in[0], A.dt[1], off[1]);
      const int64_t b = nin > 1 ? load_as_i64(A.in[1], A.dt[2], off[2]) : 0;
      store_value(A.out, A.dt[0], off[0], 0.0f, apply_i64(op, a, b), false);
    } else if (op == OPX_COPY && is_int_dt(A.dt[0]) && is_int_dt(A.dt[1])) {
      store_value(A.out, A.dt[0], off[0], 0.0f, load_as_i64(A.in[0], A.dt[1], off[1]), false);
    } else {
      const float a = load_as_f32(A.in[0], A.dt[1], off[1]);
      const float b = (nin > 1 && A.in[1]) ? load_as_f32(A.in[1], A.dt[2], off[2]) : 0.0f;
      const float c = (nin > 2 && A.in[2]) ? load_as_f32(A.in[2], A.dt[3], off[3]) : 0.0f;
      store_value(A.out, A.dt[0], off[0], apply_runtime_f32(op, a, b, c, A.alpha, A.aux), 0, true);
    }
  }
}

// ------------------------------------------------------------- launching
static int grid_for(int64_t items) {
  // Up to 32 blocks of 256 threads per CU in flight; the grid-stride loop
  // covers anything larger.
  const int64_t cap = static_cast<int64_t>(ctx().num_cus > 0 ? ctx().num_cus : 256) * 32;
  int64_t g = ceil_div(items, 256);
  if (g < 1) g = 1;
  return static_cast<int>(g < cap ? g : cap);
}

// Largest |offset| any operand reaches, to decide whether 32-bit indexing
// is safe.
static bool fits_u32(const Plan& p) {
  if (p.n >= (int64_t(1) << 31)) return false;
  for (int k = 0; k < p.nops; ++k) {
    int64_t m = 0;
    for (int d = 0; d < p.rank; ++d) {
      if (p.st[k][d] < 0) return false;
      m += (p.dims[d] - 1) * p.st[k][d];
    }
    if (m >= (int64_t(1) << 31)) return false;
  }
  return true;
}

template <int OP, int NIN>
static int launch_inner_op(const EwArgs& A, int vec, bool u32, int flat_kinds) {
  const int64_t items = A.n / vec;
  hipStream_t s = ctx().stream;
  if (flat_kinds >= 0) {
    KK_LAUNCH((ew_flat4<OP, NIN>), dim3(grid_for(A.n / 4)), dim3(256), 0, s, A,
                       flat_kinds);
    return check_launch("ew_flat4");
  }
  const int64_t per_row = A.dims[A.rank - 1] / vec;
  if (A.rank <= 2 && per_row >= 64) {
    const int64_t rows = A.rank == 2 ? A.dims[0] : 1;
    const int64_t gx = std::min<int64_t>(ceil_div(per_row, 256), 1 << 20);
    const int64_t gy = std::min<int64_t>(rows, 65535);
    const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
    if (vec == 4) KK_LAUNCH((ew_rows<OP, NIN, 4>), grid, dim3(256), 0, s, A);
    else KK_LAUNCH((ew_rows<OP, NIN, 1>), grid, dim3(256), 0, s, A);
    return check_launch("ew_rows");
  }
  const int grid = grid_for(items);
  if (vec == 4) {
    if (u32) KK_LAUNCH((ew_inner<OP, NIN, 4, uint32_t>), dim3(grid), dim3(256), 0, s, A);
    else KK_LAUNCH((ew_inner<OP, NIN, 4, int64_t>), dim3(grid), dim3(256), 0, s, A);
  } else {
    if (u32) KK_LAUNCH((ew_inner<OP, NIN, 1, uint32_t>), dim3(grid), dim3(256), 0, s, A);
    else KK_LAUNCH((ew_inner<OP, NIN, 1, int64_t>), dim3(grid), dim3(256), 0, s, A);
  }
  return check_launch("ew_inner");
}

static int launch_inner(const EwArgs& A, int nin, int vec, bool u32, int flat_kinds) {
  switch (A.op) {
#define KK_U(OPC) case OPC: return launch_inner_op<OPC, 1>(A, vec, u32, flat_kinds);
#define KK_B(OPC) case OPC: return launch_inner_op<OPC, 2>(A, vec, u32, flat_kinds);
#define KK_T(OPC) case OPC: return launch_inner_op<OPC, 3>(A, vec, u32, flat_kinds);
    KK_B(KK_OP_ADD) KK_B(KK_OP_SUB) KK_B(KK_OP_MUL) KK_B(KK_OP_DIV) KK_B(KK_OP_POW)
    KK_B(KK_OP_MIN) KK_B(KK_OP_MAX)
    KK_U(KK_OP_SQRT) KK_U(KK_OP_EXP) KK_U(KK_OP_SIN) KK_U(KK_OP_COS) KK_U(KK_OP_ATAN)
    KK_U(KK_OP_TANH) KK_U(KK_OP_SIGMOID) KK_U(KK_OP_FLOOR) KK_U(KK_OP_ROUND)
    KK_U(KK_OP_LEAKYRELU) KK_U(KK_OP_NEG) KK_U(KK_OP_ABS) KK_U(KK_OP_LOG) KK_U(KK_OP_ERF)
    KK_U(KK_OP_IDENTITY) KK_U(OPX_COPY)
    KK_T(OPX_SNAKE) KK_B(OPX_SNAKE_ALPHA) KK_B(OPX_FASTGELU) KK_U(OPX_FASTGELU_NB)
    KK_T(OPX_DEQUANT) KK_T(OPX_CLIP)
#undef KK_U
#undef KK_B
#undef KK_T
  }
  (void)nin;
  return set_error(KK_E_UNSUPPORTED, "no fast elementwise kernel for op %d", A.op);
}

static bool has_inner(int op) {
  switch (op) {
    case KK_OP_ADD: case KK_OP_SUB: case KK_OP_MUL: case KK_OP_DIV: case KK_OP_POW:
    case KK_OP_MIN: case KK_OP_MAX: case KK_OP_SQRT: case KK_OP_EXP: case KK_OP_SIN:
    case KK_OP_COS: case KK_OP_ATAN: case KK_OP_TANH: case KK_OP_SIGMOID: case KK_OP_FLOOR:
    case KK_OP_ROUND: case KK_OP_LEAKYRELU: case KK_OP_NEG: case KK_OP_ABS: case KK_OP_LOG:
    case KK_OP_ERF: case KK_OP_IDENTITY: case OPX_COPY: case OPX_SNAKE: case OPX_SNAKE_ALPHA:
    case OPX_FASTGELU: case OPX_FASTGELU_NB: case OPX_DEQUANT: case OPX_CLIP:
      return true;
  }
  return false;
}

// Plans and launches one elementwise op over `out` and up to three inputs
// (NULL entries allowed for optional operands).
static int run_elementwise(int op, const kk_tensor* out, const kk_tensor* const* ins, int nin,
                           float alpha, int aux, int mode) {
  KK_TRY(require_ready());
  KK_TRY(check_tensor(out, "out"));
  for (int k = 0; k < nin; ++k)
    if (ins[k]) KK_TRY(check_tensor(ins[k], "input"));
  Plan p;
  KK_TRY(make_plan(&p, out, ins, nin));
  if (p.n == 0) return KK_OK;
  EwArgs A;
  A.rank = p.rank;
  A.op = op;
  A.alpha = alpha;
  A.aux = aux;
  A.n = p.n;
  A.out = out->data;
  A.dt[0] = out->dtype;
  for (int k = 0; k < kMaxOperands - 1; ++k) {
    A.in[k] = (k < nin && ins[k]) ? ins[k]->data : nullptr;
    A.dt[k + 1] = (k < nin && ins[k]) ? ins[k]->dtype : KK_F32;
  }
  for (int d = 0; d < kMaxArgRank; ++d) {
    A.dims[d] = d < p.rank ? p.dims[d] : 1;
    for (int k = 0; k < kMaxOperands; ++k) A.st[k][d] = d < p.rank ? p.st[k][d] : 0;
  }
  // Fast path: every operand present and fp32, innermost stride 0 or 1 (the
  // output's must be 1).
  bool fast = mode == MODE_FLOAT && has_inner(op) && out->dtype == KK_F32 &&
              p.st[0][p.rank - 1] == 1;
  for (int k = 0; k < nin && fast; ++k) {
    if (!ins[k] || ins[k]->dtype != KK_F32) fast = false;
    else if (p.st[k + 1][p.rank - 1] != 0 && p.st[k + 1][p.rank - 1] != 1) fast = false;
  }
  if (fast) {
    const int64_t L = p.dims[p.rank - 1];
    bool vec4 = (L % 4) == 0;
    for (int k = 0; k < p.nops && vec4; ++k) {
      const void* ptr = k == 0 ? out->data : ins[k - 1]->data;
      if (p.st[k][p.rank - 1] == 0) continue;  // broadcast along rows: scalar load
      if (reinterpret_cast<uintptr_t>(ptr) % 16) vec4 = false;
      for (int d = 0; d < p.rank - 1; ++d)
        if (p.st[k][d] % 4) vec4 = false;
    }
    // The flat float4 walk, when the output is contiguous and every input
    // is contiguous like it or per-row: for rows that are not whole float4s,
    // and for rows whose float4s leave ew_rows' 256-wide column blocks more
    // than 5% idle ([1,512,2400]: 600 float4s a row, three blocks of which
    // the last has 88 of 256 lanes busy) -- the flat walk packs every lane.
    const int64_t per_row4 = L / 4;
    const bool rows_idle = vec4 && p.rank == 2 &&
                           (ceil_div(per_row4, 256) * 256 - per_row4) * 20 > per_row4;
    int kinds = -1;
    if ((!vec4 || rows_idle) && p.rank <= 2 && L >= 4 && p.n >= 4096 &&
        reinterpret_cast<uintptr_t>(out->data) % 16 == 0 &&
        (p.rank == 1 || p.st[0][0] == L)) {
      kinds = 0;
      for (int k = 0; k < nin && kinds >= 0; ++k) {
        const int64_t s1 = p.st[k + 1][p.rank - 1];
        const int64_t s0 = p.rank == 2 ? p.st[k + 1][0] : 0;
        if (s1 == 1 && (p.rank == 1 || s0 == L) &&
            reinterpret_cast<uintptr_t>(ins[k]->data) % 16 == 0) {
          continue;  // flat
        } else if (s1 == 0) {
          kinds |= 1 << (2 * k);  // per-row (or scalar)
        } else {
          kinds = -1;
        }
      }
    }
    return launch_inner(A, nin, vec4 ? 4 : 1, fits_u32(p), kinds);
  }
  KK_LAUNCH(ew_generic, dim3(grid_for(p.n)), dim3(256), 0, ctx().stream, A, nin, mode);
  return check_launch("ew_generic");
}

// ----------------------------------------------------------------- gather
// out[o, j, i] = data[o, idx[j], i] over contiguous data/out; `elem` bytes
// are moved per element (a bit-exact copy whatever the dtype).
template <typename T>
__global__ void __launch_bounds__(256) gather_kernel(T* __restrict__ out, const T* __restrict__ data,
                                                     const void* __restrict__ idx, int idx_dt,
                                                     int64_t outer, int64_t dim, int64_t nidx,
                                                     int64_t inner) {
  const int64_t n = outer * nidx * inner;
  for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < n;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i = t % inner;
    const int64_t r = t / inner;
    const int64_t j = r % nidx;
    const int64_t o = r / nidx;
    int64_t k = idx_dt == KK_I64 ? static_cast<const int64_t*>(idx)[j]
                                 : static_cast<int64_t>(static_cast<const int32_t*>(idx)[j]);
    if (k < 0) k += dim;
    k = k < 0 ? 0 : (k >= dim ? dim - 1 : k);
    out[t] = data[(o * dim + k) * inner + i];
  }
}

// A copy between two contiguous tensors of one dtype, 16-byte aligned: each
// block moves a contiguous stretch of 256 * U 16-byte items, every thread
// issuing its U non-temporal loads before its U stores (U items in flight a
// lane; one item a lane leaves a wave waiting on a single round trip); the
// last bytes % 16 are moved by block 0.
template <int U>
__global__ void __launch_bounds__(256) copy_flat16(float* __restrict__ out,
                                                   const float* __restrict__ in, int64_t n16,
                                                   int64_t tail_bytes) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (256 * U) + threadIdx.x;
  float4 v[U];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const int64_t i = base + j * 256;
    if (i < n16) v[j] = ld_stream4(in + 4 * i);
  }
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const int64_t i = base + j * 256;
    if (i < n16) st_stream4(out + 4 * i, v[j]);
  }
  if (blockIdx.x == 0 && threadIdx.x < tail_bytes) {
    const uint8_t* src = reinterpret_cast<const uint8_t*>(in + 4 * n16);
    reinterpret_cast<uint8_t*>(out + 4 * n16)[threadIdx.x] = src[threadIdx.x];
  }
}

}  // namespace kk

using namespace kk;

// Snake over rows: x and out [rows, L] (fp32, L % 4 == 0, rows xs / os
// floats apart, 16-byte aligned), alpha and recip (or 1 / alpha) one value
// per row (fp32 or fp16).  A block of up to 256 threads spans one float4 a
// thread of one row, its row's parameters loaded once (scalar loads), with
// none of the generic kernels' per-lane broadcast loads and index walk.
// Two or four float4 a thread (fewer, longer waves) measured slower at
// every decoder shape: the matching copy's speed needs the many short waves
// whose sines overlap the later waves' loads.  The same operations as
// apply_f32<OPX_SNAKE(_ALPHA)>, so the same bits.
struct SnakeRowArgs {
  float* out;
  const float* x;
  const void* alpha;
  const void* recip;
  int a_dt, r_dt;
  int64_t a_st, r_st, xs, os;
  int per_row4;
};

template <bool RECIP>
__global__ void __launch_bounds__(256) snake_rows(SnakeRowArgs S) {
  const int64_t row = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= S.per_row4) return;
  const float al = load_as_f32(S.alpha, S.a_dt, row * S.a_st);
  const float rc = RECIP ? load_as_f32(S.recip, S.r_dt, row * S.r_st) : 1.0f / al;
  const float4 v = ld_stream4(S.x + row * S.xs + 4 * static_cast<int64_t>(i));
  const float a[4] = {v.x, v.y, v.z, v.w};
  float r[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = a[e] + rc * kk_sin_sq(al * a[e]);
  st_stream4(S.out + row * S.os + 4 * static_cast<int64_t>(i), make_float4(r[0], r[1], r[2], r[3]));
}

// The row kernel when the operands have its layout; false, launching
// nothing, otherwise.
static bool snake_rows_try(const kk_tensor* out, const kk_tensor* x, const kk_tensor* alpha,
                           const kk_tensor* recip, int* status) {
  if (x->dtype != KK_F32 || out->dtype != KK_F32) return false;
  if (!(alpha->dtype == KK_F32 || alpha->dtype == KK_F16)) return false;
  if (recip && !(recip->dtype == KK_F32 || recip->dtype == KK_F16)) return false;
  const kk_tensor* ins[3] = {x, alpha, recip};
  Plan p;
  if (make_plan(&p, out, ins, recip ? 3 : 2) != KK_OK || p.n == 0 || p.rank > 2) return false;
  const int last = p.rank - 1;
  const int64_t L = p.dims[last], rows = p.rank == 2 ? p.dims[0] : 1;
  if (L % 4 || L / 4 >= (int64_t{1} << 30) || rows > 65535) return false;
  if (p.st[0][last] != 1 || p.st[1][last] != 1 || p.st[2][last] != 0) return false;
  if (recip && p.st[3][last] != 0) return false;
  const int64_t os = p.rank == 2 ? p.st[0][0] : 0, xs = p.rank == 2 ? p.st[1][0] : 0;
  if (os % 4 || xs % 4 || (reinterpret_cast<uintptr_t>(out->data) & 15) ||
      (reinterpret_cast<uintptr_t>(x->data) & 15))
    return false;
  SnakeRowArgs S{static_cast<float*>(out->data), static_cast<const float*>(x->data), alpha->data,
                 recip ? recip->data : nullptr, alpha->dtype, recip ? recip->dtype : KK_F32,
                 p.rank == 2 ? p.st[2][0] : 0, recip && p.rank == 2 ? p.st[3][0] : 0, xs, os,
                 static_cast<int>(L / 4)};
  const int width = static_cast<int>(std::min<int64_t>(256, ceil_div(L / 4, 64) * 64));
  const dim3 grid(static_cast<unsigned>(ceil_div(L / 4, int64_t{width})), static_cast<unsigned>(rows));
  if (recip) KK_LAUNCH((snake_rows<true>), grid, dim3(width), 0, ctx().stream, S);
  else KK_LAUNCH((snake_rows<false>), grid, dim3(width), 0, ctx().stream, S);
  *status = check_launch("snake_rows");
  return true;
}

extern "C" {

int kk_binary(int op, const kk_tensor* out, const kk_tensor* a, const kk_tensor* b) {
  KK_TRY(check_tensor(a, "a"));
  KK_TRY(check_tensor(b, "b"));
  const kk_tensor* ins[2] = {a, b};
  const bool cmp = op >= KK_OP_EQUAL && op <= KK_OP_AND;
  switch (op) {
    case KK_OP_ADD: case KK_OP_SUB: case KK_OP_MUL: case KK_OP_DIV: case KK_OP_POW:
    case KK_OP_MIN: case KK_OP_MAX: case KK_OP_EQUAL: case KK_OP_GREATER: case KK_OP_LESS:
    case KK_OP_GEQ: case KK_OP_AND:
      break;
    default:
      return set_error(KK_E_ARG, "kk_binary: op %d is not binary", op);
  }
  if (cmp) {
    if (out->dtype != KK_BOOL) return set_error(KK_E_ARG, "kk_binary: comparison output must be bool");
    return run_elementwise(op, out, ins, 2, 0.0f, 0, MODE_DOUBLE);
  }
  const bool fa = is_float(a->dtype), fb = is_float(b->dtype);
  if (fa && fb) {
    if (!is_float(out->dtype)) return set_error(KK_E_ARG, "kk_binary: float inputs need a float output");
    return run_elementwise(op, out, ins, 2, 0.0f, 0, MODE_FLOAT);
  }
  if (!fa && !fb) {
    if (op == KK_OP_POW) return set_error(KK_E_UNSUPPORTED, "kk_binary: integer Pow");
    if (is_float(out->dtype)) return set_error(KK_E_ARG, "kk_binary: integer inputs need an integer output");
    return run_elementwise(op, out, ins, 2, 0.0f, 0, MODE_INT);
  }
  return set_error(KK_E_UNSUPPORTED, "kk_binary: mixed float/integer operands (dtypes %d, %d)",
                   a->dtype, b->dtype);
}

int kk_unary(int op, const kk_tensor* out, const kk_tensor* x, float alpha) {
  KK_TRY(check_tensor(x, "x"));
  const kk_tensor* ins[1] = {x};
  switch (op) {
    case KK_OP_SQRT: case KK_OP_EXP: case KK_OP_SIN: case KK_OP_COS: case KK_OP_ATAN:
    case KK_OP_TANH: case KK_OP_SIGMOID: case KK_OP_FLOOR: case KK_OP_ROUND:
    case KK_OP_LEAKYRELU: case KK_OP_LOG: case KK_OP_ERF:
      if (!is_float(x->dtype) || !is_float(out->dtype))
        return set_error(KK_E_ARG, "kk_unary: op %d needs float input and output", op);
      return run_elementwise(op, out, ins, 1, alpha, 0, MODE_FLOAT);
    case KK_OP_NEG: case KK_OP_ABS: case KK_OP_IDENTITY:
      return run_elementwise(op, out, ins, 1, alpha, 0, is_float(x->dtype) ? MODE_FLOAT : MODE_INT);
  }
  return set_error(KK_E_ARG, "kk_unary: op %d is not unary", op);
}

int kk_where(const kk_tensor* out, const kk_tensor* cond, const kk_tensor* x, const kk_tensor* y) {
  KK_TRY(check_tensor(cond, "cond"));
  KK_TRY(check_tensor(x, "x"));
  KK_TRY(check_tensor(y, "y"));
  const kk_tensor* ins[3] = {cond, x, y};
  const bool fl = is_float(out->dtype);
  return run_elementwise(OPX_WHERE, out, ins, 3, 0.0f, 0, fl ? MODE_FLOAT : MODE_INT);
}

int kk_clip(const kk_tensor* out, const kk_tensor* x, const kk_tensor* lo, const kk_tensor* hi) {
  KK_TRY(check_tensor(x, "x"));
  if (!is_float(x->dtype) || !is_float(out->dtype))
    return set_error(KK_E_UNSUPPORTED, "kk_clip: float tensors only");
  const kk_tensor* ins[3] = {x, lo, hi};
  const int aux = (lo ? 1 : 0) | (hi ? 2 : 0);
  if (!lo && !hi) {
    const kk_tensor* one[1] = {x};
    return run_elementwise(OPX_COPY, out, one, 1, 0.0f, 0, MODE_FLOAT);
  }
  if (!lo || !hi) {
    // The fast path wants every operand present: stand the missing bound in
    // with x itself, whose flag bit is off.
    ins[1] = lo ? lo : x;
    ins[2] = hi ? hi : x;
  }
  return run_elementwise(OPX_CLIP, out, ins, 3, 0.0f, aux, MODE_FLOAT);
}

int kk_snake(const kk_tensor* out, const kk_tensor* x, const kk_tensor* alpha,
             const kk_tensor* recip) {
  KK_TRY(check_tensor(x, "x"));
  KK_TRY(check_tensor(alpha, "alpha"));
  if (!is_float(x->dtype) || !is_float(alpha->dtype) || out->dtype != KK_F32)
    return set_error(KK_E_ARG, "kk_snake: float tensors only, fp32 output");
  if (recip) KK_TRY(check_tensor(recip, "recip"));
  KK_TRY(require_ready());
  KK_TRY(check_tensor(out, "out"));
  int st = KK_OK;
  if (snake_rows_try(out, x, alpha, recip, &st)) return st;
  if (recip) {
    const kk_tensor* ins[3] = {x, alpha, recip};
    return run_elementwise(OPX_SNAKE, out, ins, 3, 0.0f, 0, MODE_FLOAT);
  }
  const kk_tensor* ins[2] = {x, alpha};
  return run_elementwise(OPX_SNAKE_ALPHA, out, ins, 2, 0.0f, 0, MODE_FLOAT);
}

int kk_fast_gelu(const kk_tensor* out, const kk_tensor* x, const kk_tensor* bias) {
  KK_TRY(check_tensor(x, "x"));
  if (!is_float(x->dtype) || out->dtype != KK_F32)
    return set_error(KK_E_ARG, "kk_fast_gelu: float tensors only, fp32 output");
  if (bias) {
    KK_TRY(check_tensor(bias, "bias"));
    const kk_tensor* ins[2] = {x, bias};
    return run_elementwise(OPX_FASTGELU, out, ins, 2, 0.0f, 0, MODE_FLOAT);
  }
  // Without a bias numpy skips the add entirely (so -0.0 stays -0.0).
  const kk_tensor* ins[1] = {x};
  return run_elementwise(OPX_FASTGELU_NB, out, ins, 1, 0.0f, 0, MODE_FLOAT);
}

int kk_dequantize(const kk_tensor* out, const kk_tensor* q, const kk_tensor* scale,
                  const kk_tensor* zp) {
  KK_TRY(check_tensor(q, "q"));
  KK_TRY(check_tensor(scale, "scale"));
  if (out->dtype != KK_F32) return set_error(KK_E_ARG, "kk_dequantize: fp32 output");
  const kk_tensor* ins[3] = {q, scale, zp};
  return run_elementwise(OPX_DEQUANT, out, ins, 3, 0.0f, 0, MODE_FLOAT);
}

int kk_copy(const kk_tensor* out, const kk_tensor* x) {
  KK_TRY(check_tensor(x, "x"));
  KK_TRY(check_tensor(out, "out"));
  if (out->dtype == x->dtype && out->rank == x->rank && is_contiguous(out) &&
      is_contiguous(x) && numel(out) == numel(x) && numel(x) > 0 &&
      reinterpret_cast<uintptr_t>(out->data) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(x->data) % 16 == 0) {
    bool same = true;
    for (int d = 0; d < x->rank; ++d) same = same && out->shape[d] == x->shape[d];
    if (same) {
      KK_TRY(require_ready());
      const int64_t bytes = numel(x) * dtype_size(x->dtype);
      // Four items a lane between 16 and 64 MB, one elsewhere (measured on
      // MI355X, eager launches over inputs rotating past the Infinity Cache:
      // 4.9 MB 2.97 us with one item against 3.48 with four; 39 MB 7.11 us
      // with four against 7.87; 73 MB 23.7 against 26.3; 220 MB 66.5 against
      // 73.8).
      const int U = bytes > (int64_t{16} << 20) && bytes < (int64_t{64} << 20) ? 4 : 1;
      const int64_t n16 = bytes / 16;
      const int64_t blocks = std::max<int64_t>(1, ceil_div(n16, 256 * U));
      if (blocks >= (int64_t(1) << 31))
        return set_error(KK_E_UNSUPPORTED, "kk_copy: %lld bytes exceed one launch",
                         (long long)bytes);
      float* o = static_cast<float*>(out->data);
      const float* in = static_cast<const float*>(x->data);
      if (U == 4)
        KK_LAUNCH((copy_flat16<4>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, ctx().stream,
                  o, in, n16, bytes - 16 * n16);
      else
        KK_LAUNCH((copy_flat16<1>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, ctx().stream,
                  o, in, n16, bytes - 16 * n16);
      return check_launch("copy_flat16");
    }
  }
  const kk_tensor* ins[1] = {x};
  const int mode = (is_float(out->dtype) || is_float(x->dtype)) ? MODE_FLOAT : MODE_INT;
  return run_elementwise(OPX_COPY, out, ins, 1, 0.0f, 0, mode);
}

__global__ void fill_kernel(EwArgs A, double value) {
  const int64_t n = A.n;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t rem = i, off = 0;
    for (int d = A.rank - 1; d >= 0; --d) {
      const int64_t coord = rem % A.dims[d];
      rem /= A.dims[d];
      off += coord * A.st[0][d];
    }
    const bool f = A.dt[0] == KK_F32 || A.dt[0] == KK_F16 || A.dt[0] == KK_BOOL;
    store_value(A.out, A.dt[0], off, static_cast<float>(value), static_cast<int64_t>(value), f);
  }
}

int kk_fill(const kk_tensor* out, double value) {
  KK_TRY(require_ready());
  KK_TRY(check_tensor(out, "out"));
  Plan p;
  KK_TRY(make_plan(&p, out, nullptr, 0));
  if (p.n == 0) return KK_OK;
  EwArgs A;
  A.rank = p.rank;
  A.n = p.n;
  A.out = out->data;
  A.dt[0] = out->dtype;
  for (int d = 0; d < kMaxArgRank; ++d) {
    A.dims[d] = d < p.rank ? p.dims[d] : 1;
    A.st[0][d] = d < p.rank ? p.st[0][d] : 0;
  }
  KK_LAUNCH(fill_kernel, dim3(grid_for(p.n)), dim3(256), 0, ctx().stream, A, value);
  return check_launch("fill_kernel");
}

int kk_gather(const kk_tensor* out, const kk_tensor* data, const kk_tensor* indices, int axis) {
  KK_TRY(require_ready());
  KK_TRY(check_tensor(out, "out"));
  KK_TRY(check_tensor(data, "data"));
  KK_TRY(check_tensor(indices, "indices"));
  if (data->rank < 1) return set_error(KK_E_ARG, "kk_gather: data must have rank >= 1");
  if (axis < 0) axis += data->rank;
  if (axis < 0 || axis >= data->rank) return set_error(KK_E_ARG, "kk_gather: axis out of range");
  if (!is_contiguous(data) || !is_contiguous(indices) || !is_contiguous(out))
    return set_error(KK_E_ARG, "kk_gather: data, indices and out must be contiguous");
  if (indices->dtype != KK_I64 && indices->dtype != KK_I32)
    return set_error(KK_E_ARG, "kk_gather: indices must be int32/int64");
  if (out->dtype != data->dtype) return set_error(KK_E_ARG, "kk_gather: out dtype must match data");
  // Expected output shape: data[:axis] + indices + data[axis+1:].
  const int orank = data->rank - 1 + indices->rank;
  if (out->rank != orank) return set_error(KK_E_ARG, "kk_gather: output rank %d, expected %d", out->rank, orank);
  int j = 0;
  for (int i = 0; i < axis; ++i, ++j)
    if (out->shape[j] != data->shape[i]) return set_error(KK_E_ARG, "kk_gather: output shape mismatch");
  for (int i = 0; i < indices->rank; ++i, ++j)
    if (out->shape[j] != indices->shape[i]) return set_error(KK_E_ARG, "kk_gather: output shape mismatch");
  for (int i = axis + 1; i < data->rank; ++i, ++j)
    if (out->shape[j] != data->shape[i]) return set_error(KK_E_ARG, "kk_gather: output shape mismatch");
  int64_t outer = 1, inner = 1;
  for (int i = 0; i < axis; ++i) outer *= data->shape[i];
  for (int i = axis + 1; i < data->rank; ++i) inner *= data->shape[i];
  const int64_t dim = data->shape[axis];
  const int64_t nidx = numel(indices);
  const int64_t n = outer * nidx * inner;
  if (n == 0) return KK_OK;
  if (dim == 0) return set_error(KK_E_ARG, "kk_gather: cannot index an empty axis");
  const int grid = grid_for(n);
  hipStream_t s = ctx().stream;
  switch (dtype_size(data->dtype)) {
    case 1:
      KK_LAUNCH(gather_kernel<uint8_t>, dim3(grid), dim3(256), 0, s,
                         static_cast<uint8_t*>(out->data), static_cast<const uint8_t*>(data->data),
                         indices->data, indices->dtype, outer, dim, nidx, inner);
      break;
    case 2:
      KK_LAUNCH(gather_kernel<uint16_t>, dim3(grid), dim3(256), 0, s,
                         static_cast<uint16_t*>(out->data), static_cast<const uint16_t*>(data->data),
                         indices->data, indices->dtype, outer, dim, nidx, inner);
      break;
    case 4:
      KK_LAUNCH(gather_kernel<uint32_t>, dim3(grid), dim3(256), 0, s,
                         static_cast<uint32_t*>(out->data), static_cast<const uint32_t*>(data->data),
                         indices->data, indices->dtype, outer, dim, nidx, inner);
      break;
    default:
      KK_LAUNCH(gather_kernel<uint64_t>, dim3(grid), dim3(256), 0, s,
                         static_cast<uint64_t*>(out->data), static_cast<const uint64_t*>(data->data),
                         indices->data, indices->dtype, outer, dim, nidx, inner);
  }
  return check_launch("gather_kernel");
}

}  // extern "C"
