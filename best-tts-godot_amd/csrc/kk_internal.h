// Internal declarations shared by the libkk translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <type_traits>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "kk.h"

namespace kk {

// ---------------------------------------------------------------- context
struct Context {
  bool ready = false;
  int device = -1;
  hipStream_t stream = nullptr;
  int num_cus = 0;
  bool capturing = false;  // between kk_graph_begin and kk_graph_end
  // Per-row arrival counters of the multi-block row reductions, zero
  // between launches (the last block of a row resets its counter), then
  // kFlagSlots per-call slots, each cleared by the call that uses it before
  // it is set.
  int* row_counters = nullptr;
  // Device scratch owned by the context from kk_init to kk_shutdown, for
  // per-call intermediates that must not be allocated (calls recorded into
  // graphs): every call runs on the one stream, so each use is finished
  // before the next call's kernels run, and the buffer never moves while a
  // recorded graph may refer to it.
  void* scratch = nullptr;
  // Kernels launched outside graph recording since kk_init (each replay of a
  // recorded graph launches its kernels without passing through here).
  uint64_t dispatches = 0;
};
constexpr size_t kScratchBytes = size_t{16} << 20;
constexpr int kRowCounters = 65536;
constexpr int kFlagSlots = 64;

// DynamicQuantizeLinear's byte of x with the scale rounded to fp32 and the
// zero point as a float: clamp(rint(x / scale) + zp, 0, 255)
// (ref_runtime.py:106-116; the sum of two integers is exact in fp32).
__device__ __forceinline__ uint32_t dql_byte(float x, float sc, float z) {
  float v = rintf(x / sc) + z;
  v = v < 0.0f ? 0.0f : (v > 255.0f ? 255.0f : v);
  return static_cast<uint32_t>(v);
}

// Scale and zero point from the (min, max) of x, in double exactly as the
// reference does; returns (scale, zero point) as floats (x / scale runs in
// float32 against the scale rounded to float32) and stores the outputs.
__device__ inline float2 dql_params(float fmn, float fmx, float* scale_out, uint8_t* zp_out) {
  const double mn = fmn;
  const double mx = fmx;
  const double dlo = mn < 0.0 ? mn : 0.0;
  const double dhi = mx > 0.0 ? mx : 0.0;
  double scale = (dhi - dlo) / 255.0;
  if (scale == 0.0) scale = 1.0;
  double zp = rint(0.0 - dlo / scale);
  zp = zp < 0.0 ? 0.0 : (zp > 255.0 ? 255.0 : zp);
  *scale_out = static_cast<float>(scale);
  *zp_out = static_cast<uint8_t>(zp);
  return make_float2(static_cast<float>(scale), static_cast<float>(zp));
}

// Folds npart (min, max) partials and derives DynamicQuantizeLinear's scale
// and zero point: params[0] = (scale, zp) as floats, *scale_out, *zp_out.
// With only_if, the launch does nothing unless *only_if == epoch; with
// clear, params[1] = the folded (min, max) and *clear = 0.
int launch_dql_fold(const float2* part, int npart, float2* params, float* scale_out,
                    uint8_t* zp_out, const int* only_if = nullptr, int* clear = nullptr,
                    int epoch = 0);
Context& ctx();
// Every kernel launch of the library goes through KK_LAUNCH, which counts it
// (kk_dispatch_count) unless a graph is being recorded.
#define KK_LAUNCH(...)                                        \
  do {                                                        \
    if (!::kk::ctx().capturing) ++::kk::ctx().dispatches;     \
    hipLaunchKernelGGL(__VA_ARGS__);                          \
  } while (0)
// Takes the device address of the allocation-free convolution's file-scope
// scratch for `device` (current), once per device (kk_conv_i8.hip).
int conv_i8_scratch_setup(int device);
// Drops the record of what a packed ConvInteger weight buffer at `p` was
// made from (kk_free calls it: the address may next hold anything).
void conv_i8_forget_pack(const void* p);
// The same for a packed fp16 matrix-core convolution weight (kk_conv_f16.hip).
void convh_forget_pack(const void* p);
void gemm_forget_pack(const void* p);
// Leaf sums a convolution formed of its [rows, T] fp32 output x, for the
// InstanceNorm that reads x (kk_free forgets the record of either buffer).
void leaf_record(const void* leaf, const void* x, int64_t rows, int64_t T);
bool leaf_matches(const void* leaf, const void* x, int64_t rows, int64_t T);
// Drops the record of what a packed MatMulInteger B at `p` was made from
// (kk_free calls it).
void i8_forget_pack(const void* p);

// Thread-local last error; set_error returns `code` so call sites can
// `return set_error(KK_E_ARG, "...")`.
int set_error(int code, const char* fmt, ...);
int check_hip(hipError_t e, const char* what);
int require_ready();

#define KK_TRY(expr)            \
  do {                          \
    int _rc = (expr);           \
    if (_rc != KK_OK) return _rc; \
  } while (0)

#define KK_HIP(expr) KK_TRY(::kk::check_hip((expr), #expr))

// Checks the launch that was just enqueued.
int check_launch(const char* kernel);

// ------------------------------------------------------------ descriptors
int dtype_size(int dtype);
bool is_float(int dtype);
bool is_int(int dtype);
int64_t numel(const kk_tensor* t);
bool is_contiguous(const kk_tensor* t);
// Validates rank, dtype and non-negative extents; `name` goes in the error.
int check_tensor(const kk_tensor* t, const char* name);

// An elementwise plan: up to four operands (0 = output) walked over one
// collapsed index space.  Strides are in elements, broadcast axes carry 0.
constexpr int kMaxOperands = 4;
struct Plan {
  int rank = 0;
  int64_t dims[KK_MAX_RANK];
  int64_t st[kMaxOperands][KK_MAX_RANK];
  int nops = 0;
  int64_t n = 0;
};
// Broadcasts the inputs against out->shape (numpy right alignment), drops
// unit axes and merges adjacent axes that every operand walks contiguously
// (the same rule as runtime/ops.gd:85-129).  ins may hold NULL entries,
// which are skipped (their strides stay 0).
int make_plan(Plan* p, const kk_tensor* out, const kk_tensor* const* ins,
              int nins);

// -------------------------------------------------------- device helpers
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Wave-wide sum / max through DPP lane moves instead of the butterfly's six
// ds_bpermute round trips through LDS: pairs (quad_perm 1,0,3,2), quads
// (quad_perm 2,3,0,1), half rows (row_half_mirror), rows of 16
// (row_mirror), then rows 0+1 and 2+3 (row_bcast15 into rows 1 and 3) and
// all four (row_bcast31 into rows 2 and 3); lane 63 ends with the total,
// which readlane makes wave-uniform.  A different (fixed) order of additions
// than wave_sum: for kernels held to a tolerance, not to numpy's bits.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_move(float v, float fill) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(v), CTRL,
                                                    ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = v + dpp_move<0xB1, 0xF>(v, 0.0f);
  v = v + dpp_move<0x4E, 0xF>(v, 0.0f);
  v = v + dpp_move<0x141, 0xF>(v, 0.0f);
  v = v + dpp_move<0x140, 0xF>(v, 0.0f);
  v = v + dpp_move<0x142, 0xA>(v, 0.0f);
  v = v + dpp_move<0x143, 0xC>(v, 0.0f);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_move<0xB1, 0xF>(v, -INFINITY));
  v = fmaxf(v, dpp_move<0x4E, 0xF>(v, -INFINITY));
  v = fmaxf(v, dpp_move<0x141, 0xF>(v, -INFINITY));
  v = fmaxf(v, dpp_move<0x140, 0xF>(v, -INFINITY));
  v = fmaxf(v, dpp_move<0x142, 0xA>(v, -INFINITY));
  v = fmaxf(v, dpp_move<0x143, 0xC>(v, -INFINITY));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Streaming (non-temporal) 128-bit and 32-bit accesses for data that is
// read or written once per kernel.  Several 16-byte stores per thread with
// ordinary write-back stores measured 3-5x slower on MI355X than the same
// pattern with non-temporal stores.
typedef float kk_f4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_stream4(const float* p) {
  const kk_f4v v = __builtin_nontemporal_load(reinterpret_cast<const kk_f4v*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_stream4(float* p, float4 v) {
  const kk_f4v t = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(t, reinterpret_cast<kk_f4v*>(p));
}
__device__ __forceinline__ float ld_stream(const float* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_stream(float* p, float v) { __builtin_nontemporal_store(v, p); }

// Loads element `i` of a buffer of dtype `dt` as fp32 (fp16 is storage only).
__device__ __forceinline__ float load_as_f32(const void* p, int dt, int64_t i) {
  switch (dt) {
    case KK_F32: return static_cast<const float*>(p)[i];
    case KK_F16: return __half2float(static_cast<const __half*>(p)[i]);
    case KK_I8: return static_cast<float>(static_cast<const int8_t*>(p)[i]);
    case KK_U8: return static_cast<float>(static_cast<const uint8_t*>(p)[i]);
    case KK_I32: return static_cast<float>(static_cast<const int32_t*>(p)[i]);
    case KK_I64: return static_cast<float>(static_cast<const int64_t*>(p)[i]);
    case KK_BOOL: return static_cast<const uint8_t*>(p)[i] ? 1.0f : 0.0f;
  }
  return 0.0f;
}

__device__ __forceinline__ int64_t load_as_i64(const void* p, int dt, int64_t i) {
  switch (dt) {
    case KK_I8: return static_cast<const int8_t*>(p)[i];
    case KK_U8: return static_cast<const uint8_t*>(p)[i];
    case KK_I32: return static_cast<const int32_t*>(p)[i];
    case KK_I64: return static_cast<const int64_t*>(p)[i];
    case KK_BOOL: return static_cast<const uint8_t*>(p)[i] ? 1 : 0;
    case KK_F32: return static_cast<int64_t>(static_cast<const float*>(p)[i]);
    case KK_F16:
      return static_cast<int64_t>(__half2float(static_cast<const __half*>(p)[i]));
  }
  return 0;
}

// Weight dequantisation parameters shared by gemm, conv and adain: a
// per-tensor or per-column scale and zero point, read once on the host side
// of the launch as device pointers.
struct Dequant {
  const void* scale = nullptr;  // fp32/fp16, 1 or `count` elements
  int scale_dt = KK_F32;
  int64_t scale_stride = 0;     // 0 = per tensor
  const void* zp = nullptr;     // int8/uint8/int32, 1 or `count` elements
  int zp_dt = KK_I8;
  int64_t zp_stride = 0;
  bool active = false;          // true for int8/uint8 weights
};
// Checks `w_scale`/`w_zp` against the weight dtype and the number of
// columns (`count`) they may be indexed by.
int make_dequant(Dequant* d, const kk_tensor* w, const kk_tensor* scale,
                 const kk_tensor* zp, int64_t count, const char* who);

__device__ __forceinline__ float dequant_value(float q, const Dequant& d,
                                               int64_t col) {
  float z = d.zp ? load_as_f32(d.zp, d.zp_dt, col * d.zp_stride) : 0.0f;
  if (!d.scale) return q - z;  // integer ops: zero-point shift only
  float s = load_as_f32(d.scale, d.scale_dt, col * d.scale_stride);
  return (q - z) * s;
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// sin(t) in fp32 for the Sin node and every fused snake: t = k pi + r with
// k = rint(t / pi) and r from three FMA steps against pi = P1 + P2 + P3
// (Cody and Waite's additive reduction; k is below 2^15, so each k * Pi
// term is formed exactly inside its FMA), then the odd Taylor series of sin
// to r^13 (|r| <= pi/2: the first term left out is below 7e-10), negated
// for odd k.  Measured against float64 sin on 45,000 arguments up to 1e4:
// within 1.7 ulp.  |t| > 1e5 (and inf, NaN) take the library sinf; a zero
// keeps its sign.
__device__ __forceinline__ float kk_sin(float t) {
  if (!(fabsf(t) <= 1.0e5f)) return sinf(t);
  const float k = rintf(t * 0x1.45f306p-2f) + 0.0f;  // 1/pi; + 0 turns -0 into +0
  float r = __builtin_fmaf(-k, 0x1.921fb6p+1f, t);
  r = __builtin_fmaf(-k, -0x1.777a5cp-24f, r);
  r = __builtin_fmaf(-k, -0x1.ee58p-49f, r);
  const float r2 = r * r;
  float p = 0x1.612462p-33f;                     //  1/13!
  p = __builtin_fmaf(p, r2, -0x1.ae6456p-26f);   // -1/11!
  p = __builtin_fmaf(p, r2, 0x1.71de3ap-19f);    //  1/9!
  p = __builtin_fmaf(p, r2, -0x1.a01a02p-13f);   // -1/7!
  p = __builtin_fmaf(p, r2, 0x1.111112p-7f);     //  1/5!
  p = __builtin_fmaf(p, r2, -0x1.555556p-3f);    // -1/3!
  const float s = __builtin_fmaf(r2 * r, p, r);
  const float v = (static_cast<int>(k) & 1) ? -s : s;
  return t == 0.0f ? t : v;
}

// kk_sin(t) * kk_sin(t), bit for bit, for the snake: squaring drops the sign,
// so the odd-k negation, the signed-zero return and k's -0 -> +0 are not
// needed (they only change the sign of the sine: +-s and +-0 square to the
// same bits).
__device__ __forceinline__ float kk_sin_sq(float t) {
  if (!(fabsf(t) <= 1.0e5f)) {
    const float s = sinf(t);
    return s * s;
  }
  const float k = rintf(t * 0x1.45f306p-2f);
  float r = __builtin_fmaf(-k, 0x1.921fb6p+1f, t);
  r = __builtin_fmaf(-k, -0x1.777a5cp-24f, r);
  r = __builtin_fmaf(-k, -0x1.ee58p-49f, r);
  const float r2 = r * r;
  float p = 0x1.612462p-33f;
  p = __builtin_fmaf(p, r2, -0x1.ae6456p-26f);
  p = __builtin_fmaf(p, r2, 0x1.71de3ap-19f);
  p = __builtin_fmaf(p, r2, -0x1.a01a02p-13f);
  p = __builtin_fmaf(p, r2, 0x1.111112p-7f);
  p = __builtin_fmaf(p, r2, -0x1.555556p-3f);
  const float s = __builtin_fmaf(r2 * r, p, r);
  return s * s;
}

// exp(x) for x <= 0 (softmax's x - max): 2^(x log2 e) on the hardware
// exp2, with the rounding error of the product x * log2(e) recovered by an
// FMA (and log2(e)'s own low part) and applied as 2^e ~ 1 + e ln 2.  Within
// a few ulp of the correctly rounded exp over [-87, 0] (results below 2^-126
// flush to 0); exp(0) = 1 exactly.
__device__ __forceinline__ float kk_exp_neg(float x) {
  const float t = x * 0x1.715476p+0f;                   // log2(e), rounded
  const float e = __builtin_fmaf(x, 0x1.715476p+0f, -t) + x * 0x1.4ae0bep-26f;
  return __builtin_amdgcn_exp2f(t) * __builtin_fmaf(e, 0x1.62e430p-1f, 1.0f);  // ln 2
}

// a / b for many a over one divisor b, bit-identical to the division: with
// rb = 1 / b correctly rounded, q0 = a * rb, the exact remainder
// r = fma(-q0, b, a) and q = fma(r, rb, q0) is a / b correctly rounded
// (Markstein's theorem: P. Markstein, IBM J. Res. Dev. 34(1), 1990) when no
// step underflows or overflows, which 2^-60 <= b <= 2^60 and
// 2^-60 < |a| < 2^60 guarantee.  Three instructions and two compares against
// the division's ten; other divisors (rb = 0) and dividends (zeros, tiny or
// huge values, inf, NaN) take the division itself.
struct KkDivisor {
  float b, rb;
};
__device__ __forceinline__ KkDivisor kk_divisor(float b) {
  return KkDivisor{b, (b >= 0x1p-60f && b <= 0x1p60f) ? 1.0f / b : 0.0f};
}
__device__ __forceinline__ float kk_div_fast(float a, const KkDivisor& d) {
  const float q0 = a * d.rb;
  return __builtin_fmaf(__builtin_fmaf(-q0, d.b, a), d.rb, q0);
}
// (the tests are combined with & rather than &&: short-circuit evaluation
// compiles to a branch per test)
__device__ __forceinline__ int kk_div_in_range(float a) {
  const float m = __builtin_fabsf(a);
  return static_cast<int>(m > 0x1p-60f) & static_cast<int>(m < 0x1p60f);
}
__device__ __forceinline__ float kk_div(float a, const KkDivisor& d) {
  float q = kk_div_fast(a, d);
  if (!(static_cast<int>(d.rb != 0.0f) & kk_div_in_range(a))) q = a / d.b;
  return q;
}
// Four quotients; the divisions run only where one of the four is out of range.
__device__ __forceinline__ float4 kk_div4(float4 a, const KkDivisor& d) {
  float4 q = make_float4(kk_div_fast(a.x, d), kk_div_fast(a.y, d), kk_div_fast(a.z, d),
                         kk_div_fast(a.w, d));
  const int ok = static_cast<int>(d.rb != 0.0f) & kk_div_in_range(a.x) & kk_div_in_range(a.y) &
                 kk_div_in_range(a.z) & kk_div_in_range(a.w);
  if (!ok) q = make_float4(a.x / d.b, a.y / d.b, a.z / d.b, a.w / d.b);
  return q;
}

// DynamicQuantizeLinear's bytes of four values, dql_byte's rounding with
// the quotients x / scale formed by kk_div4 (the same bits), packed
// little-endian.
__device__ __forceinline__ uint32_t dql_byte_of_quotient(float q, float z) {
  float v = rintf(q) + z;
  v = v < 0.0f ? 0.0f : (v > 255.0f ? 255.0f : v);
  return static_cast<uint32_t>(v);
}
__device__ __forceinline__ uint32_t dql_bytes4(float4 x, const KkDivisor& sc, float z) {
  const float4 q = kk_div4(x, sc);
  return dql_byte_of_quotient(q.x, z) | (dql_byte_of_quotient(q.y, z) << 8) |
         (dql_byte_of_quotient(q.z, z) << 16) | (dql_byte_of_quotient(q.w, z) << 24);
}

// Runs f(integral_constant<U>, t + U) for U = 0 .. R - 1 while t + U < end:
// a loop body written out R times, so that a register ring indexed by U
// keeps constant indices (a runtime index would put the ring in scratch).
template <int U, int R>
struct Unroll {
  template <class F>
  __device__ __forceinline__ static void run(F& f, int t, int end) {
    if (t + U >= end) return;
    f(std::integral_constant<int, U>{}, t + U);
    Unroll<U + 1, R>::run(f, t, end);
  }
};
template <int R>
struct Unroll<R, R> {
  template <class F>
  __device__ __forceinline__ static void run(F&, int, int) {}
};

// Batch offsets of a batched matmul: up to 6 batch axes with per-operand
// strides (0 = broadcast).
struct BatchMap {
  int nb = 0;
  int64_t dims[6];
  int64_t st[3][6];  // 0 = a, 1 = b, 2 = out
};

__device__ __forceinline__ int64_t batch_offset(const BatchMap& bm, int which, int64_t b) {
  int64_t off = 0;
  for (int d = bm.nb - 1; d >= 0; --d) {
    off += (b % bm.dims[d]) * bm.st[which][d];
    b /= bm.dims[d];
  }
  return off;
}

// Shapes of out = a @ w under numpy's matmul rules (rank >= 2 operands,
// batch axes broadcast): fills *bm and M, N, K and the batch count.
int matmul_shape(const kk_tensor* out, const kk_tensor* a, const kk_tensor* w, BatchMap* bm,
                 int64_t* M, int64_t* N, int64_t* K, int64_t* batch, const char* who);
// kk_gemm; weights_rounded keeps numpy's rounding of each dequantised weight
// (the fp32 matrix cores) where a caller's result feeds a recurrence.
// `packed` (checked here): w laid out by kk_gemm_pack, used where the bf16
// matrix-core path takes the call (the same results as without it).
int gemm(const kk_tensor* out, const kk_tensor* a, const kk_tensor* w, const kk_tensor* w_scale,
         const kk_tensor* w_zp, float alpha, bool weights_rounded,
         const kk_tensor* packed = nullptr);
// out = A @ dequant(B) on the bf16 matrix cores (kk_gemm_dq.hip) when the
// operands fit: fp32 A with K contiguous, int8/uint8 B (zero point of the
// same type) or fp16 B with N contiguous.  Returns false, launching nothing,
// when they do not; *status is the launch's status otherwise.
bool gemm_dq_try(const float* a, int64_t a_si, const void* b, int b_dt, int64_t b_si,
                 const Dequant& dq, float* out, int64_t som, int64_t son, const BatchMap& bm,
                 int64_t M, int64_t N, int64_t K, int64_t batch, float alpha, const int* only_if,
                 const void* bpack, int* status);
// kk_gemm_pack's layout: its size, the check of a packed buffer against a
// call, and the registry entry dropped when the buffer is freed.
int64_t gemm_packed_size(int64_t K, int64_t N, int w_dt);
int gemm_check_packed(const kk_tensor* packed, const kk_tensor* w, const kk_tensor* w_zp,
                      const char* who);
void gemm_forget_pack(const void* p);
// XCD-aware block order (this library is built for gfx950 alone, whose
// parts have 8 XCDs): workgroup w runs on XCD w % 8, so XCD x is given
// the contiguous run of tiles x q + min(x, r) .. (T = 8 q + r tiles, the
// first r XCDs one more), x-fastest: neighbouring tiles, which share input
// rows or halos, share an L2.  A bijection on the grid; the tile's (x, y, z).
__device__ inline uint3 xcd_tile() {
  const uint32_t gx = gridDim.x, gy = gridDim.y;
  const uint32_t tiles = gx * gy * gridDim.z;
  const uint32_t wid = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const uint32_t xcd = wid % 8u, q8 = tiles / 8u, r8 = tiles % 8u;
  const uint32_t t = xcd * q8 + (xcd < r8 ? xcd : r8) + wid / 8u;
  return make_uint3(t % gx, (t / gx) % gy, t / (gx * gy));
}
// Host check for a grid whose kernel calls xcd_tile: its block count, and
// so every linear block id, fits the 32-bit arithmetic above.
inline int check_xcd_grid(const dim3& g, const char* who) {
  const uint64_t n = uint64_t{g.x} * g.y * g.z;
  if (n >= (uint64_t{1} << 32))
    return set_error(KK_E_UNSUPPORTED, "%s: %llu blocks exceed the 32-bit tile order", who,
                     static_cast<unsigned long long>(n));
  return KK_OK;
}

// A zero-point-only shift (scale 1) for the integer ops: per tensor, or per
// element of `count` when the zero point has that many elements.
int zp_shift(Dequant* d, const kk_tensor* zp, int64_t count, const char* who);



}  // namespace kk
