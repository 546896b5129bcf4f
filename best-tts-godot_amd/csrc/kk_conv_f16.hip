// Conv1d and ConvTranspose1d with fp16 or 8-bit weights on the fp16 matrix
// cores (v_mfma_f32_32x32x16_f16), fp32 results, in one launch.
//
// Exact operands.  An fp16 weight is exact in fp16, and so is an 8-bit
// weight less its zero point (|q - zp| <= 255); the 8-bit weights' scale,
// per tensor or per output channel, multiplies the fp32 sum
// (sum (q - zp) s x = s sum (q - zp) x up to fp32 rounding).  Every output
// column (time step) scales its activations by its own power of two, 2^k,
// chosen from the largest |x| its receptive field has shown so far: with m
// that maximum, m 2^k first lies in [2^10, 2^11) (exact in fp32), and a
// scaled y = x 2^k is split into hi = fp16(y) and lo = fp16(y - hi) (y - hi
// is exact in fp32).  For |y| >= 2^-3 lo is a normal fp16 number and hi + lo
// equals y to within 2^-22 |y|; below that the error is at most 2^-25 in
// scaled units, m 2^-35 or less.  Every product w hi and w lo is exact in
// fp32 (11 + 11 significant bits) and the matrix cores accumulate them in
// fp32.  Only when a column's maximum grows past 2^15 in scaled units (a
// value 16 to 32 times the first maximum) does its k fall afresh; its
// accumulators (all in the lanes that hold that column) are then multiplied
// by 2^(k_new - k_old), exact for a power of two.  The sums are scaled back
// by 2^-k at the end.  A column whose receptive field holds an infinity or
// a NaN is recomputed with scalar fp32 products and sums, which give numpy's
// inf / NaN pattern.
//
// Both operations are one implicit GEMM with rows m = co P + r (output
// channel co, phase r < P) and columns q, the reduction index k running over
// (input channel ci, tap t') with TP in {2, 4, 8} taps a channel (T taps
// used, the rest weigh 0):
//   out[co, q os + r + oph] = sum_ci sum_t' Wv[m][ci][t'] x[ci, q qs + ta + t' tm]
//   Conv1d (P = 1): t' = the tap, qs = stride, ta = -pad0, tm = dilation,
//     os = 1, oph = 0, Wv[co][ci][t'] = W[co][ci][t'].
//   ConvTranspose1d (dilation 1), P = stride phases, T = ceil(K / P) taps a
//     phase, read in increasing position: x[ci, q - (T - 1) + t'] (qs = 1,
//     ta = 1 - T, tm = 1), os = stride, oph = -pad0,
//     Wv[co P + r][ci][t'] = W[ci][co][r + P (T - 1 - t')] (0 past K).
// A 16-deep reduction slice s holds channels 16 s / TP .. + 16 / TP - 1, each
// with its TP taps, so a lane's eight operand values of a slice are TP
// consecutive taps of 8 / TP channels: for Conv1d with dilation 1 and for
// ConvTranspose1d, consecutive x positions of each channel.
//
// Packed weights (kk_conv_pack, or per call into the context scratch): fp16
// values (W less its zero point) in the matrix cores' operand order: the
// 16-byte unit (mt KS + s) 64 + l holds lane l's operand of slice s for rows
// 32 mt .. 32 mt + 31: row 32 mt + l % 32, k = 8 (l / 32) + 0..7 (KS slices;
// zeros past M, past Cin and past T).
//
// A block owns 32 MI rows x 32 WN columns; its 4 waves are WN (columns) x
// WK (reduction ranges).  A wave holds MI 32 x 32 accumulator tiles of its
// 32 columns: lane (n, g) = (lane % 32, lane / 32) loads its column's eight
// x values of a slice straight from memory (bounds-checked buffer loads: 0
// outside the signal, past Cin and past T), the two lanes of a column agree
// on its scale (one lane swap), and split, and the weights' operands come
// as 1 KB fragments; both run three slices ahead in a register ring, with
// no LDS and no barrier in the reduction loop.  The WK waves of a column
// range add their unscaled partial tiles through LDS in wave order.
#include <algorithm>
#include <climits>
#include <mutex>
#include <unordered_map>

#include "kk_internal.h"

namespace kk {
namespace convh {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;

// Taps a channel spans in the reduction order: T rounded up to 2, 4 or 8 (0:
// more than 8 taps, which this path does not take).
static int taps_padded(int64_t T) { return T <= 2 ? 2 : T <= 4 ? 4 : T <= 8 ? 8 : 0; }

// The packed geometry: what a pack and a convolution must agree on.
struct Geo {
  int transposed;
  int64_t Cin, Cout, Kw, P;  // P: phases (the stride) of a transposed conv, else 1
  int64_t T, TP;             // taps a row reads; taps a channel spans (0: unsupported)
  int64_t M, MT, KS;         // rows, 32-row tiles, 16-deep slices
  int64_t bytes;             // packed size
};

static Geo geometry(bool transposed, int64_t Cin, int64_t Cout, int64_t Kw, int64_t stride) {
  Geo g{};
  g.transposed = transposed ? 1 : 0;
  g.Cin = Cin; g.Cout = Cout; g.Kw = Kw;
  g.P = transposed ? stride : 1;
  g.T = transposed ? ceil_div(Kw, stride) : Kw;
  g.TP = taps_padded(g.T);
  g.M = g.P * Cout;
  g.MT = ceil_div(g.M, 32);
  g.KS = g.TP ? ceil_div(Cin * g.TP, 16) : 0;
  g.bytes = g.MT * g.KS * 1024;
  return g;
}

struct PackArgs {
  uint4* wp;
  const void* w;   // conv [Cout][Cin][Kw], transposed [Cin][Cout][Kw]
  const void* zp;  // 8-bit weights' zero point (1 or Cout values) or NULL
  int zp_dt;
  int zp_stride;
  int Cin, Cout, Kw, P, T, TP, M, KS;
  int transposed;
  int64_t units;
};

// One 16-byte unit (eight fp16 values) a thread.
template <typename TW>
__global__ void __launch_bounds__(256) convh_pack(PackArgs A) {
  const int64_t u = blockIdx.x * int64_t{256} + threadIdx.x;
  if (u >= A.units) return;
  const int l = static_cast<int>(u % 64);
  const int s = static_cast<int>((u / 64) % A.KS);
  const int mt = static_cast<int>(u / (int64_t{64} * A.KS));
  const int m = 32 * mt + (l % 32), g = l / 32;
  const int co = m / A.P, r = m - co * A.P;
  const TW* w = static_cast<const TW*>(A.w);
  const float z = A.zp && m < A.M ? load_as_f32(A.zp, A.zp_dt, co * A.zp_stride) : 0.0f;
  h8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = 8 * g + e;
    const int ci = s * (16 / A.TP) + k / A.TP, tp = k % A.TP;
    const int tap = A.transposed ? r + A.P * (A.T - 1 - tp) : tp;
    float f = 0.0f;
    if (m < A.M && ci < A.Cin && tp < A.T && tap < A.Kw) {
      const int64_t idx = A.transposed ? (static_cast<int64_t>(ci) * A.Cout + co) * A.Kw + tap
                                       : (static_cast<int64_t>(co) * A.Cin + ci) * A.Kw + tap;
      f = static_cast<float>(w[idx]) - z;
    }
    v[e] = static_cast<_Float16>(f);
  }
  *reinterpret_cast<h8*>(A.wp + u) = v;
}

struct CArgs {
  const uint4* wp;     // packed weights
  const float* x;      // [N][Cin][L]
  float* out;          // [N][Cout][Lout]
  const float* bias;   // [Cout] or NULL
  const void* scale;   // 8-bit weights: 1 or Cout values; NULL for fp16 weights
  int scale_dt, scale_stride;
  int Cin, L, Cout, Lout, M, Nq, P, T, KS;
  int qs, ta, tm;      // x position of (q, t'): q qs + ta + t' tm
  int os, oph;         // output position of (q, r): q os + r + oph
  int wbytes;          // packed bytes (below 2^31)
};

// The power of two k with m 2^k in [2^10, 2^11) for the bits of m = max |x|
// > 0, kept within [-120, 120] so that 2^k and 2^-k are normal floats.
__device__ __forceinline__ int scale_exp(unsigned mbits) {
  const int e = static_cast<int>(mbits >> 23) - 127;  // floor(log2 m); -127 for subnormal m
  return min(120, 10 - e);
}

template <int TP, int MI, int WK, int R>
__global__ void __launch_bounds__(kThreads) convh_kernel(CArgs A) {
  constexpr int WN = 4 / WK, CPL = 8 / TP, CPS = 16 / TP;
  constexpr int BM = 32 * MI, BN = 32 * WN;
  constexpr int RED = WK > 1 ? (WK - 1) * WN * MI * 16 * 64 : 1;
  __shared__ float red[RED];       // [wk - 1][wn][register][lane]: the other waves' partials
  __shared__ int red_bad[4 * 64];  // [wave][lane]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave % WN, wk = wave / WN;
  const int ln = lane & 31, g = lane >> 5;
  // row tiles fastest: the blocks of one column range share an XCD.  The
  // tile is wave-uniform; readfirstlane says so to the compiler, which would
  // otherwise build the activations' buffer resource in vector registers
  // and wrap every load in a loop over its distinct values.
  const uint3 tile = xcd_tile();
  const int m0 = __builtin_amdgcn_readfirstlane(static_cast<int>(tile.x)) * BM;
  const int n0 = __builtin_amdgcn_readfirstlane(static_cast<int>(tile.y)) * BN;
  const int64_t b = __builtin_amdgcn_readfirstlane(static_cast<int>(tile.z));
  const int Cin = A.Cin, L = A.L, KS = A.KS;
  const int q = n0 + wn * 32 + ln;
  const int s0 = static_cast<int>(static_cast<int64_t>(KS) * wk / WK);
  const int ns = static_cast<int>(static_cast<int64_t>(KS) * (wk + 1) / WK) - s0;
  const auto xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(A.x + b * Cin * L), 0,
                                                     Cin * L * 4, 0x00020000);
  const auto wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint4*>(A.wp), 0, A.wbytes,
                                                     0x00020000);
  // byte offsets of this lane's TP positions in a channel row; 0x7fffffff
  // outside the signal, past the columns or past the T taps in use, and a
  // channel's offset 0x80000000 past Cin: any sum with either is past the
  // buffer (below 2^31 bytes), so the load returns 0, and no sum wraps
  uint32_t po[TP];
#pragma unroll
  for (int t = 0; t < TP; ++t) {
    const int p = q * A.qs + A.ta + t * A.tm;
    po[t] = q < A.Nq && t < A.T && p >= 0 && p < L ? static_cast<uint32_t>(4 * p) : 0x7fffffffu;
  }
  const int row_bytes = 4 * L;
  const uint32_t a_lane = static_cast<uint32_t>(((m0 / 32) * KS * 64 + lane) * 16);
  // per-row epilogue constants (output row offset, phase offset, scale,
  // bias), filled by the first BM threads; read after the block's barrier
  __shared__ int4 rows[BM];
  if (tid < BM) {
    const int m = m0 + tid;
    int4 rv = make_int4(-1, 0, __float_as_int(1.0f), 0);
    if (m < A.M) {
      const int co = m / A.P, r = m - co * A.P;
      rv.x = co * A.Lout;
      rv.y = r + A.oph;
      if (A.scale) rv.z = __float_as_int(load_as_f32(A.scale, A.scale_dt, co * A.scale_stride));
      if (A.bias) rv.w = __float_as_int(A.bias[co]);
    }
    rows[tid] = rv;
  }
  float bv[R][8];
  uint4 av[R][MI];
  // slice s's x values (channels s CPS + g CPL + c, each with its TP taps)
  // and weight fragments; issued whatever s (a read past the buffers
  // returns 0), so every slot's loads count the same for the waits
  auto fetch = [&](int s, float (&v)[8], uint4 (&f)[MI]) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ci = s * CPS + g * CPL + c;
      const uint32_t cofs = ci < Cin ? static_cast<uint32_t>(ci * row_bytes) : 0x80000000u;
#pragma unroll
      for (int t = 0; t < TP; ++t) {
        uint32_t off = cofs + po[t];
        asm volatile("" : "+v"(off));  // an unconditional load
        v[c * TP + t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xrs, off, 0, 0));
      }
    }
    const uint32_t a_s = a_lane + static_cast<uint32_t>(s * 1024);
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      uint32_t off = a_s + static_cast<uint32_t>(mi * KS * 1024);
      asm volatile("" : "+v"(off));
      const auto r = __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 0);
      f[mi] = make_uint4(r[0], r[1], r[2], r[3]);
    }
  };

  f16v acc[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
  int kcur = 0, have = 0, bad = 0;
  // one slice: the column's running scale, the split, the products
  auto mma = [&](float (&v)[8], const uint4 (&f)[MI]) {
    unsigned mx = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = max(mx, __float_as_uint(v[e]) & 0x7fffffffu);
    const auto pr = __builtin_amdgcn_permlane32_swap(mx, mx, false, false);  // the column's other lane
    mx = max(static_cast<unsigned>(pr[0]), static_cast<unsigned>(pr[1]));
    const bool nonfinite = mx >= 0x7f800000u;
    if (nonfinite) {
      bad = 1;  // recomputed in the epilogue; no products from this slice
    } else if (mx != 0u) {
      if (!have) {
        kcur = scale_exp(mx);
        have = 1;
      } else if (static_cast<int>(mx >> 23) - 127 + kcur >= 15) {  // m 2^k >= 2^15
        const int kc = scale_exp(mx);
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][r] = ldexpf(acc[i][r], kc - kcur);
        kcur = kc;
      }
    }
    const float xs = nonfinite ? 0.0f : ldexpf(1.0f, kcur);
    h8 hi, lo;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float y = v[e] * xs;  // |y| < 2^15: exact
      const _Float16 hh = static_cast<_Float16>(y);
      hi[e] = hh;
      lo[e] = static_cast<_Float16>(y - static_cast<float>(hh));
    }
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      const h8 a = __builtin_bit_cast(h8, f[mi]);
      acc[mi] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, hi, acc[mi], 0, 0, 0);
      acc[mi] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, lo, acc[mi], 0, 0, 0);
    }
  };
#pragma unroll
  for (int u = 0; u < R; ++u) fetch(s0 + u, bv[u], av[u]);
  // whole rounds of R slices (a slot's refill is issued whether or not its
  // slice exists: a skipped refill leaves the waits at "all loads")
  for (int i = 0; i < ns; i += R) {
#pragma unroll
    for (int u = 0; u < R; ++u) {
      if (i + u < ns) mma(bv[u], av[u]);
      fetch(s0 + i + u + R, bv[u], av[u]);
    }
  }
  const float uns = ldexpf(1.0f, -kcur);  // exact: a power of two
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] *= uns;
  if constexpr (WK > 1) {
    if (wk > 0) {
      float* dst = red + ((wk - 1) * WN + wn) * MI * 16 * 64 + lane;
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) dst[(i * 16 + r) * 64] = acc[i][r];
    }
    red_bad[wave * 64 + lane] = bad;
  }
  __syncthreads();  // the partials and the row constants
  if (wk > 0) return;
  if constexpr (WK > 1) {
#pragma unroll
    for (int k = 1; k < WK; ++k) {  // in wave order
      const float* src = red + ((k - 1) * WN + wn) * MI * 16 * 64 + lane;
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] += src[(i * 16 + r) * 64];
      bad |= red_bad[(k * WN + wn) * 64 + lane];
    }
  }
  // D(i, j) of a 32x32 tile: lane j + 32 ((i / 4) % 2), register (i / 8) 4 + i % 4.
  // Stores through a buffer resource over this item's output: an offset
  // past it (a row past M, a column past Nq, a position outside [0, Lout))
  // drops the store.
  const auto ors = __builtin_amdgcn_make_buffer_rsrc(A.out + b * A.Cout * A.Lout, 0,
                                                     A.Cout * A.Lout * 4, 0x00020000);
  const int qpos = q < A.Nq ? q * A.os : INT_MIN / 2;
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int rg = 0; rg < 16; ++rg) {
      const int ml = 32 * mi + 8 * (rg / 4) + 4 * g + (rg % 4);
      const int4 rv = rows[ml];
      const int pos = qpos + rv.y;
      const bool ok = rv.x >= 0 && pos >= 0 && pos < A.Lout;
      uint32_t off = ok ? static_cast<uint32_t>(4 * (rv.x + pos)) : 0x80000000u;
      const float u = acc[mi][rg] * __int_as_float(rv.z);  // the scale (1 for fp16 weights)
      const float v = A.bias ? u + __int_as_float(rv.w) : u;
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ors, off, 0, 0);
    }
  if (bad) {
    // a column with an infinity or a NaN: scalar fp32 products and sums over
    // the packed weights (fp16 -> fp32 exact) and the raw activations give
    // numpy's inf / NaN pattern
    const float* xb = A.x + b * Cin * L;
    const _Float16* wh = reinterpret_cast<const _Float16*>(A.wp);
    for (int i = 0; i < 16 * MI; ++i) {
      const int ml = 32 * (i / 16) + 8 * ((i % 16) / 4) + 4 * g + (i % 4);
      const int m = m0 + ml;
      const int4 rv = rows[ml];
      const int pos = qpos + rv.y;
      if (m >= A.M || pos < 0 || pos >= A.Lout) continue;
      float sum = 0.0f;
      for (int ci = 0; ci < Cin; ++ci)
        for (int t = 0; t < A.T; ++t) {
          const int p = q * A.qs + A.ta + t * A.tm;
          if (p < 0 || p >= L) continue;
          const int k = (ci % CPS) * TP + t;
          const int64_t unit = (static_cast<int64_t>(m / 32) * KS + ci / CPS) * 64 + (m % 32) + 32 * (k / 8);
          sum = sum + static_cast<float>(wh[unit * 8 + k % 8]) * xb[static_cast<int64_t>(ci) * L + p];
        }
      const float u = A.scale ? sum * __int_as_float(rv.z) : sum;
      A.out[b * A.Cout * A.Lout + rv.x + pos] = A.bias ? u + __int_as_float(rv.w) : u;
    }
  }
}

// The launch shape: MI 32-row tiles a wave, WK waves a column range.
struct Shape {
  int mi, wk;
};

// 128 rows a wave when that still gives every SIMD a wave, else 64 (32 for
// at most 32 rows); then as many waves on the reduction (1, 2 or 4) as it
// takes to give every SIMD two waves, each at least three slices.
static Shape pick_shape(const CArgs& a, int64_t batch) {
  Shape s{};
  const int64_t simds = 4 * (ctx().num_cus > 0 ? ctx().num_cus : 256);
  const int64_t cols = batch * ceil_div(a.Nq, 32);
  s.mi = a.M <= 32 ? 1 : (a.M > 64 && cols * ceil_div(a.M, 128) >= simds) ? 4 : 2;
  const int64_t waves = cols * ceil_div(a.M, 32 * s.mi);
  s.wk = waves >= 2 * simds ? 1 : waves * 2 >= 2 * simds ? 2 : 4;
  while (s.wk > 1 && a.KS < 3 * s.wk) s.wk /= 2;
  return s;
}

template <int TP, int MI, int WK>
static int launch_shape(const CArgs& a, int64_t batch) {
  constexpr int BM = 32 * MI, BN = 32 * (4 / WK);
  constexpr int R = 3;  // slices in flight (six measured no faster at MI <= 2)
  const dim3 grid(static_cast<unsigned>(ceil_div(a.M, BM)), static_cast<unsigned>(ceil_div(a.Nq, BN)),
                  static_cast<unsigned>(batch));
  KK_TRY(check_xcd_grid(grid, "convh_kernel"));
  KK_LAUNCH((convh_kernel<TP, MI, WK, R>), grid, dim3(kThreads), 0, ctx().stream, a);
  return check_launch("convh_kernel");
}

template <int TP>
static int launch_tp(const CArgs& a, const Shape& s, int64_t batch) {
#define KK_CONVH_WK(MI)                                           \
  switch (s.wk) {                                                 \
    case 1: return launch_shape<TP, MI, 1>(a, batch);             \
    case 2: return launch_shape<TP, MI, 2>(a, batch);             \
    default: return launch_shape<TP, MI, 4>(a, batch);            \
  }
  if (s.mi == 1) KK_CONVH_WK(1)
  if (s.mi == 2) KK_CONVH_WK(2)
  KK_CONVH_WK(4)
#undef KK_CONVH_WK
}

static int launch(const CArgs& a, int tp, int64_t batch) {
  const Shape s = pick_shape(a, batch);
  if (tp == 2) return launch_tp<2>(a, s, batch);
  if (tp == 4) return launch_tp<4>(a, s, batch);
  return launch_tp<8>(a, s, batch);
}

// The pack of w (less its zero point) into `wp` (g.bytes, 16-byte aligned).
static int pack(const Geo& g, void* wp, const kk_tensor* w, const Dequant& dq) {
  PackArgs p{};
  p.wp = static_cast<uint4*>(wp);
  p.w = w->data;
  p.zp = dq.zp;
  p.zp_dt = dq.zp_dt;
  p.zp_stride = static_cast<int>(dq.zp_stride);
  p.Cin = static_cast<int>(g.Cin); p.Cout = static_cast<int>(g.Cout); p.Kw = static_cast<int>(g.Kw);
  p.P = static_cast<int>(g.P); p.T = static_cast<int>(g.T); p.TP = static_cast<int>(g.TP);
  p.M = static_cast<int>(g.M); p.KS = static_cast<int>(g.KS);
  p.transposed = g.transposed;
  p.units = g.bytes / 16;
  const dim3 grid(static_cast<unsigned>(ceil_div(p.units, 256)));
  if (w->dtype == KK_F16) KK_LAUNCH(convh_pack<_Float16>, grid, dim3(256), 0, ctx().stream, p);
  else if (w->dtype == KK_I8) KK_LAUNCH(convh_pack<int8_t>, grid, dim3(256), 0, ctx().stream, p);
  else KK_LAUNCH(convh_pack<uint8_t>, grid, dim3(256), 0, ctx().stream, p);
  return check_launch("convh_pack");
}

// Weights the fp16 path takes: fp16 as they are; 8-bit less an 8-bit zero
// point (the difference is an integer of at most 255: exact in fp16).
static bool weights_ok(const kk_tensor* w, const Dequant& dq) {
  const bool w16 = w->dtype == KK_F16 && !dq.active;
  const bool w8 = (w->dtype == KK_I8 || w->dtype == KK_U8) &&
                  (!dq.zp || dq.zp_dt == KK_I8 || dq.zp_dt == KK_U8);
  return w16 || w8;
}

// The launch arguments of a call, or false when the fp16 path does not
// apply (more than 8 taps, or sizes beyond its 32-bit offsets and grid).
static bool make_args(CArgs* a, const Geo& g, const kk_tensor* out, const kk_tensor* x,
                      const Dequant& dq, const kk_tensor* bias, int64_t stride, int64_t dilation,
                      int64_t pad0, int64_t Nq) {
  const int64_t N = x->shape[0], L = x->shape[2], Lout = out->shape[2];
  if (!g.TP || x->dtype != KK_F32 || N > 65535 || g.Cin * L * 4 >= (int64_t{1} << 31) ||
      g.Cout * Lout * 4 >= (int64_t{1} << 31) || g.bytes >= (int64_t{1} << 31) ||
      (Nq + 1) * std::max<int64_t>(stride, 1) + g.TP * dilation + pad0 >= (int64_t{1} << 29) ||
      (Nq + 1) * g.P + Lout + pad0 >= (int64_t{1} << 30) || g.M >= (int64_t{1} << 30))
    return false;
  *a = CArgs{};
  a->x = static_cast<const float*>(x->data);
  a->out = static_cast<float*>(out->data);
  a->bias = bias ? static_cast<const float*>(bias->data) : nullptr;
  a->scale = dq.scale;
  a->scale_dt = dq.scale_dt;
  a->scale_stride = static_cast<int>(dq.scale_stride);
  a->Cin = static_cast<int>(g.Cin); a->L = static_cast<int>(L);
  a->Cout = static_cast<int>(g.Cout); a->Lout = static_cast<int>(Lout);
  a->M = static_cast<int>(g.M); a->Nq = static_cast<int>(Nq); a->P = static_cast<int>(g.P);
  a->T = static_cast<int>(g.T); a->KS = static_cast<int>(g.KS);
  if (g.transposed) {
    a->qs = 1; a->ta = static_cast<int>(1 - g.T); a->tm = 1;
    a->os = static_cast<int>(g.P); a->oph = static_cast<int>(-pad0);
  } else {
    a->qs = static_cast<int>(stride); a->ta = static_cast<int>(-pad0); a->tm = static_cast<int>(dilation);
    a->os = 1; a->oph = 0;
  }
  a->wbytes = static_cast<int>(g.bytes);
  return true;
}

// What a packed buffer was made from (checked by every packed call).
struct PackRecord {
  const void* w;
  int64_t d0, d1, d2;
  int w_dt;
  const void* zp;
  int zp_dt;
  int transposed;
  int64_t stride;
};
static std::mutex g_pack_mu;
static std::unordered_map<const void*, PackRecord> g_packs;

static PackRecord record_of(const kk_tensor* w, const kk_tensor* w_zp, bool transposed, int64_t stride) {
  return PackRecord{w->data, w->shape[0], w->shape[1], w->shape[2], w->dtype,
                    w_zp ? w_zp->data : nullptr, w_zp ? w_zp->dtype : -1, transposed ? 1 : 0,
                    transposed ? stride : 1};
}

}  // namespace convh

using namespace convh;

void convh_forget_pack(const void* p) {
  std::lock_guard<std::mutex> lock(g_pack_mu);
  g_packs.erase(p);
}

// The fp16 matrix-core convolution of one call: true when it ran (its
// status in *rc), false when it does not apply (the caller runs the fp32
// kernels).  `packed` (checked by the caller) holds the weights laid out by
// kk_conv_pack; without it they are laid out here, in the context scratch
// (or a pooled workspace, freed after the launch in stream order).
bool convh_run(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w, const Dequant& dq,
               const kk_tensor* bias, bool transposed, int64_t stride, int64_t dilation,
               int64_t pad0, int64_t Nq, const kk_tensor* packed, int* rc) {
  *rc = KK_OK;
  if (!weights_ok(w, dq) || (transposed && dilation != 1)) return false;
  const int64_t Cin = x->shape[1];
  const int64_t Cout = out->shape[1], Kw = w->shape[2];
  const Geo g = geometry(transposed, Cin, Cout, Kw, stride);
  // enough work for the matrix cores
  if (Cin < 8 || g.M * Nq * g.T * Cin < (int64_t{1} << 24)) return false;
  CArgs a;
  if (!make_args(&a, g, out, x, dq, bias, stride, dilation, pad0, Nq)) return false;
  if (packed) {
    a.wp = static_cast<const uint4*>(packed->data);
  } else {
    void* wp = nullptr;
    void* ws = nullptr;
    if (g.bytes <= static_cast<int64_t>(kScratchBytes)) wp = ctx().scratch;
    else if (!ctx().capturing && kk_alloc(static_cast<size_t>(g.bytes), &ws) == KK_OK) wp = ws;
    if (!wp) return false;
    *rc = pack(g, wp, w, dq);
    if (*rc == KK_OK) {
      a.wp = static_cast<const uint4*>(wp);
      *rc = launch(a, static_cast<int>(g.TP), x->shape[0]);
    }
    if (ws) kk_free(ws);  // stream order keeps it alive for the kernels above
    return true;
  }
  *rc = launch(a, static_cast<int>(g.TP), x->shape[0]);
  return true;
}

// Checks a packed buffer against the call: its size and alignment, and that
// the last kk_conv_pack into it read this w (and zero point) for this
// geometry.
int convh_check_packed(const kk_tensor* packed, const kk_tensor* w, const kk_tensor* w_zp,
                       bool transposed, int64_t stride, const char* who) {
  KK_TRY(check_tensor(packed, "packed"));
  const int64_t cin = transposed ? w->shape[0] : w->shape[1];
  const int64_t cout = transposed ? w->shape[1] : w->shape[0];
  const int64_t need = geometry(transposed, cin, cout, w->shape[2], stride).bytes;
  if (packed->dtype != KK_U8 || !is_contiguous(packed) || numel(packed) != need ||
      reinterpret_cast<uintptr_t>(packed->data) % 256 != 0)
    return set_error(KK_E_ARG, "%s: packed must be %lld contiguous, 256-byte aligned uint8 bytes",
                     who, (long long)need);
  const PackRecord want = record_of(w, w_zp, transposed, stride);
  std::lock_guard<std::mutex> lock(g_pack_mu);
  auto it = g_packs.find(packed->data);
  if (it == g_packs.end()) return set_error(KK_E_ARG, "%s: packed was not made by kk_conv_pack", who);
  const PackRecord& r = it->second;
  if (r.w != want.w || r.d0 != want.d0 || r.d1 != want.d1 || r.d2 != want.d2 || r.w_dt != want.w_dt)
    return set_error(KK_E_ARG, "%s: packed was made from another weight tensor", who);
  if (r.zp != want.zp || r.zp_dt != want.zp_dt)
    return set_error(KK_E_ARG, "%s: packed was made with another weight zero point", who);
  if (r.transposed != want.transposed || r.stride != want.stride)
    return set_error(KK_E_ARG, "%s: packed was made for another %s", who,
                     r.transposed != want.transposed ? "operation" : "stride");
  return KK_OK;
}

}  // namespace kk

using namespace kk;

extern "C" {

int kk_conv_packed_bytes(int transposed, int64_t cin, int64_t cout, int64_t k, int stride,
                         int64_t* bytes) {
  if (!bytes || cin <= 0 || cout <= 0 || k <= 0 || stride < 1)
    return set_error(KK_E_ARG, "kk_conv_packed_bytes: positive sizes, stride and an output");
  const Geo g = geometry(transposed != 0, cin, cout, k, stride);
  if (!g.TP)
    return set_error(KK_E_UNSUPPORTED, "kk_conv_packed_bytes: %lld taps a row (more than 8) are "
                     "not packed", (long long)g.T);
  *bytes = g.bytes;
  return KK_OK;
}

int kk_conv_pack(const kk_tensor* packed, const kk_tensor* w, const kk_tensor* w_zp,
                 int transposed, int stride) {
  const char* who = "kk_conv_pack";
  KK_TRY(require_ready());
  KK_TRY(check_tensor(w, "w"));
  if (w->rank != 3 || !(w->dtype == KK_F16 || w->dtype == KK_I8 || w->dtype == KK_U8) ||
      !is_contiguous(w) || numel(w) == 0 || stride < 1)
    return set_error(KK_E_ARG,
                     "%s: w must be a non-empty contiguous fp16/int8/uint8 tensor of rank 3 and "
                     "stride >= 1", who);
  const bool tr = transposed != 0;
  const int64_t cin = tr ? w->shape[0] : w->shape[1];
  const int64_t cout = tr ? w->shape[1] : w->shape[0];
  Dequant dq;
  if (w_zp) {
    if (w->dtype == KK_F16) return set_error(KK_E_ARG, "%s: an fp16 weight takes no zero point", who);
    KK_TRY(check_tensor(w_zp, "w_zp"));
    if (!(w_zp->dtype == KK_I8 || w_zp->dtype == KK_U8))
      return set_error(KK_E_ARG, "%s: w_zp must be int8/uint8", who);
    KK_TRY(zp_shift(&dq, w_zp, cout, who));
  }
  const Geo g = geometry(tr, cin, cout, w->shape[2], stride);
  if (!g.TP)
    return set_error(KK_E_UNSUPPORTED, "%s: %lld taps a row (more than 8) are not packed", who,
                     (long long)g.T);
  if (g.bytes >= (int64_t{1} << 31))
    return set_error(KK_E_UNSUPPORTED, "%s: %lld packed bytes exceed 2 GiB", who, (long long)g.bytes);
  KK_TRY(check_tensor(packed, "packed"));
  if (packed->dtype != KK_U8 || !is_contiguous(packed) || numel(packed) != g.bytes ||
      reinterpret_cast<uintptr_t>(packed->data) % 256 != 0)
    return set_error(KK_E_ARG, "%s: packed must be %lld contiguous, 256-byte aligned uint8 bytes",
                     who, (long long)g.bytes);
  {
    std::lock_guard<std::mutex> lock(g_pack_mu);
    g_packs[packed->data] = record_of(w, w_zp, tr, stride);
  }
  return pack(g, packed->data, w, dq);
}

}  // extern "C"
