// Conv1d and ConvTranspose1d with fp16 or 8-bit weights on the fp16 matrix
// cores, fp32 results.
//
// An fp16 weight is exact in fp16, and so is an 8-bit weight less its zero
// point (|q - zp| <= 255); the 8-bit weights' scale, per tensor or per
// output channel, multiplies the fp32 sum (sum (q - zp) s x = s sum (q - zp) x,
// the same value up to fp32 rounding).  A first pass forms m = max |x| over
// the input; every activation is then scaled by 2^k, the power of two that
// puts m in [2^14, 2^15) (exact in fp32), and the scaled y = x 2^k is split
// into hi = fp16(y) and lo = fp16(y - hi) (y - hi is exact in fp32).  For
// |y| >= 2^-3 lo is a normal fp16 number and hi + lo equals y to within
// 2^-22 |y|; below that (|x| < m 2^-17) the error is at most 2^-25 in
// scaled units, m 2^-39 or less.  Every product w*hi and w*lo is exact in
// fp32 (11 + 11 significant bits), v_mfma_f32_32x32x16_f16 accumulates them
// in fp32, and the sum is scaled back by 2^-k (exact): the accuracy of fp32
// products accumulated in fp32, at the fp16 matrix rate, whatever the
// activations' magnitude.  A non-finite activation (m inf or NaN) sets a
// flag instead; the fp32 kernels, launched after this one with that flag as
// their condition, then compute the convolution.
//
// Both operations are one implicit GEMM with rows m = co*P + r (output
// channel co, phase r < P):
//   out[co, q*os + r + ophase0] = sum_kk Wt[m][kk] * x[ci, q*qs + t*tap_mul + tap_add]
// with kk = t*Cin + ci (tap-major, so a K-step of 32 has one tap t).
//   Conv1d (P = 1): t = the tap k, qs = stride, tap_mul = dilation,
//     tap_add = -pad0, os = 1, ophase0 = 0; Wt[co][k*Cin + ci] = W[co][ci][k].
//   ConvTranspose1d, P = stride phases (dilation 1): t = m, x[ci, q - m],
//     qs = 1, tap_mul = -1, tap_add = 0, os = stride, ophase0 = -pad0;
//     Wt[co*P + r][m*Cin + ci] = W[ci][co][r + stride*m] (0 past the kernel).
//     A block's rows hold every phase of its output channels, so its
//     stores fill whole lines of the interleaved output in its L2.
// A call rearranges W into Wt (fp16, less the zero point) first, in the
// library context's scratch (a pooled workspace when larger), so each K-step
// loads its weight rows as vectors.  A Wt beyond the scratch while a graph
// is being recorded (nothing may be allocated then) is not stored: the
// kernel gathers the same fp16 values from W itself (slower, the same
// results bit for bit).  The non-finite flag and m are slots of the library
// context, cleared at the start of each call.
#include <algorithm>

#include "kk_internal.h"

namespace kk {
namespace convh {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16v __attribute__((ext_vector_type(16)));

#ifndef KK_CONVH_BK
#define KK_CONVH_BK 32
#endif
constexpr int kBK = KK_CONVH_BK;  // K-step (halves)
constexpr int kPitch = kBK + 8;  // LDS row pitch (halves): 80 bytes
constexpr int kThreads = 256;

struct HArgs {
  const _Float16* wt;  // [M][Kg] when rearranged, else NULL
  const void* w;       // conv [Cout][Cin][Kw], transposed [Cin][Cout][Kw]
  int transposed;
  int64_t Kw, s;       // kernel taps, stride (the phase count P for transposed)
  Dequant dq;          // 8-bit weights: zero point subtracted, scale applied to the sums
  const float* x;      // [N, Cin, L]
  float* out;          // [N, Cout, Lout]
  const float* bias;   // [Cout] or NULL
  int* flag;           // set: an activation is not finite
  unsigned* xmax;      // bits of max |x| (a non-negative float, so ordered as unsigned)
  int64_t Cin, L, M, Cout, Kg, Nq, Lout;
  int64_t qs, tap_mul, tap_add, os, ophase0;
  int P;
  // split-K (ring kernel): blockIdx.z = batch * ksplit + split; each split
  // sums its share of the K-steps into part[(b * ksplit + split) * M + m][q]
  // (raw, in the activations' scaled units), NULL for the direct epilogue
  int ksplit;
  float* part;
  int64_t Mp;  // rows of the rearranged weights: M rounded up to 128 (zeros past M)
};

// WAVES_M x (4 / WAVES_M) wavefronts, each owning WM_T x WN_T tiles of 32x32.
template <int WAVES_M_, int WM_T_, int WN_T_>
struct Tile {
  static constexpr int WAVES_M = WAVES_M_, WM_T = WM_T_, WN_T = WN_T_;
  static constexpr int WAVES_N = 4 / WAVES_M;
  static constexpr int BM = WAVES_M * 32 * WM_T, BN = WAVES_N * 32 * WN_T;
  // A staging: thread -> row t % BM, KPT consecutive k from KPT * (t / BM)
  static constexpr int KPT = BM * kBK / kThreads;
  static_assert(kThreads % BM == 0 && KPT % 4 == 0, "A staging shape");
  // B staging: thread -> column n = t % BN, k pairs t / BN + j * (256 / BN)
  static constexpr int KP_STEP = kThreads / BN;
  static constexpr int B_PAIRS = (kBK / 2) / KP_STEP;
  static_assert(kThreads % BN == 0 && (kBK / 2) % KP_STEP == 0, "B staging shape");
};

// The power of two k with m 2^k in [2^14, 2^15) for m = max |x| > 0 (0 for
// m = 0), kept within [-120, 120] so that 2^k and 2^-k are normal floats.
__device__ __forceinline__ int convh_scale_exp(unsigned mbits) {
  if (mbits == 0) return 0;
  const int e = static_cast<int>(mbits >> 23) - 127;  // floor(log2 m); -127 for subnormal m
  return min(120, 14 - e);
}

// PRE: the weights come rearranged in A.wt; else gathered from A.w.
template <class T, typename TW, bool PRE>
__global__ void __launch_bounds__(kThreads) convh_kernel(HArgs A) {
  __shared__ __align__(16) _Float16 As[2][T::BM * kPitch];
  __shared__ __align__(16) _Float16 Bh[2][T::BN * kPitch];
  __shared__ __align__(16) _Float16 Bl[2][T::BN * kPitch];
  constexpr int WM_T = T::WM_T, WN_T = T::WN_T;
  const unsigned mbits = *A.xmax;
  if (mbits >= 0x7f800000u) {  // an infinite or NaN activation: the fp32 kernels compute it
    if (threadIdx.x == 0) *A.flag = 1;  // every writer stores the same 1
    return;
  }
  const int kexp = convh_scale_exp(mbits);
  const float xscale = ldexpf(1.0f, kexp), unscale = ldexpf(1.0f, -kexp);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m_w = (wave / T::WAVES_N) * 32 * WM_T, n_w = (wave % T::WAVES_N) * 32 * WN_T;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * T::BN;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * T::BM;
  const int64_t b = blockIdx.z;
  const float* xb = A.x + b * A.Cin * A.L;
  const int64_t nk = A.Kg / kBK;
  const TW* w = static_cast<const TW*>(A.w);

  // this thread's A row: m = co*P + r, and its weights' zero point
  const int am = tid % T::BM, ak = T::KPT * (tid / T::BM);
  const int64_t m_row = m0 + am;
  const int64_t a_co = m_row / A.P, a_r = m_row - a_co * A.P;
  const bool a_in = m_row < A.M;
  const float a_zp = A.dq.zp && a_in ? load_as_f32(A.dq.zp, A.dq.zp_dt, a_co * A.dq.zp_stride) : 0.0f;
  const int64_t cout = A.M / A.P;
  // step between consecutive ci in W
  const int64_t w_ci = A.transposed ? cout * A.Kw : A.Kw;

  // staging registers
  _Float16 av[T::KPT];
  float bv[T::B_PAIRS][2];
  const int bn = tid % T::BN;
  const int64_t q = n0 + bn;
  auto fetch = [&](int64_t k0) {
    const int64_t t = k0 / A.Cin, ci0 = k0 - t * A.Cin;
    if constexpr (PRE) {
      typedef _Float16 h4v __attribute__((ext_vector_type(4)));
#pragma unroll
      for (int e = 0; e < T::KPT; e += 4) {
        h4v v = {};
        if (a_in) v = *reinterpret_cast<const h4v*>(A.wt + m_row * A.Kg + k0 + ak + e);
#pragma unroll
        for (int u = 0; u < 4; ++u) av[e + u] = v[u];
      }
    } else {
      // W[co][ci][t] (conv) or W[ci][co][r + s*t] (transposed, 0 past the kernel)
      const int64_t tap = A.transposed ? a_r + A.s * t : t;
      const bool tap_in = a_in && tap < A.Kw;
      const int64_t wbase = A.transposed ? ((ci0 + ak) * cout + a_co) * A.Kw + tap
                                         : (a_co * A.Cin + ci0 + ak) * A.Kw + tap;
#pragma unroll
      for (int e = 0; e < T::KPT; ++e) {
        float v = 0.0f;
        if (tap_in) v = static_cast<float>(w[wbase + e * w_ci]) - a_zp;
        av[e] = static_cast<_Float16>(v);
      }
    }
    const int64_t pos = q * A.qs + t * A.tap_mul + A.tap_add;
    const bool in = q < A.Nq && pos >= 0 && pos < A.L;
#pragma unroll
    for (int j = 0; j < T::B_PAIRS; ++j) {
      const int kp = tid / T::BN + j * T::KP_STEP;
      const float* xr = xb + (ci0 + 2 * kp) * A.L + pos;
      bv[j][0] = in ? xr[0] : 0.0f;
      bv[j][1] = in ? xr[A.L] : 0.0f;
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int e = 0; e < T::KPT; e += 4) {
      typedef _Float16 h4 __attribute__((ext_vector_type(4)));
      *reinterpret_cast<h4*>(&As[buf][am * kPitch + ak + e]) =
          h4{av[e], av[e + 1], av[e + 2], av[e + 3]};
    }
#pragma unroll
    for (int j = 0; j < T::B_PAIRS; ++j) {
      const int kp = tid / T::BN + j * T::KP_STEP;
      h2 hi, lo;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float v = bv[j][e] * xscale;  // |v| < 2^15: exact
        const _Float16 h = static_cast<_Float16>(v);
        hi[e] = h;
        lo[e] = static_cast<_Float16>(v - static_cast<float>(h));
      }
      *reinterpret_cast<h2*>(&Bh[buf][bn * kPitch + 2 * kp]) = hi;
      *reinterpret_cast<h2*>(&Bl[buf][bn * kPitch + 2 * kp]) = lo;
    }
  };

  f16v acc[WM_T][WN_T];
#pragma unroll
  for (int i = 0; i < WM_T; ++i)
#pragma unroll
    for (int j = 0; j < WN_T; ++j)
#pragma unroll
      for (int g = 0; g < 16; ++g) acc[i][j][g] = 0.0f;

  fetch(0);
  stash(0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int buf = static_cast<int>(kt & 1);
    const bool more = kt + 1 < nk;
    if (more) fetch((kt + 1) * kBK);
#pragma unroll
    for (int ks = 0; ks < kBK; ks += 16) {
      const int kofs = ks + 8 * (lane >> 5);
      h8 a[WM_T], bh[WN_T], bl[WN_T];
#pragma unroll
      for (int i = 0; i < WM_T; ++i)
        a[i] = *reinterpret_cast<const h8*>(&As[buf][(m_w + 32 * i + (lane & 31)) * kPitch + kofs]);
#pragma unroll
      for (int j = 0; j < WN_T; ++j) {
        bh[j] = *reinterpret_cast<const h8*>(&Bh[buf][(n_w + 32 * j + (lane & 31)) * kPitch + kofs]);
        bl[j] = *reinterpret_cast<const h8*>(&Bl[buf][(n_w + 32 * j + (lane & 31)) * kPitch + kofs]);
      }
#pragma unroll
      for (int i = 0; i < WM_T; ++i)
#pragma unroll
        for (int j = 0; j < WN_T; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bh[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bl[j], acc[i][j], 0, 0, 0);
        }
    }
    if (more) stash(buf ^ 1);
    __syncthreads();
  }
  // D(i, j) of a 32x32 tile: lane j + 32 * ((i / 4) % 2), register (i / 8) * 4 + i % 4
  float* ob = A.out + b * A.Cout * A.Lout;
#pragma unroll
  for (int i = 0; i < WM_T; ++i)
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      const int64_t m = m0 + m_w + 32 * i + 8 * (g / 4) + 4 * (lane >> 5) + (g % 4);
      if (m >= A.M) continue;
      const int64_t co = m / A.P, r = m - co * A.P;
      const float bias = A.bias ? A.bias[co] : 0.0f;
      const float sc = A.dq.scale ? load_as_f32(A.dq.scale, A.dq.scale_dt, co * A.dq.scale_stride)
                                  : 1.0f;
#pragma unroll
      for (int j = 0; j < WN_T; ++j) {
        const int64_t qq = n0 + n_w + 32 * j + (lane & 31);
        const float u = acc[i][j][g] * unscale;  // exact: a power of two
        const float v = A.dq.scale ? u * sc : u;
        const int64_t pos = qq * A.os + r + A.ophase0;
        if (qq < A.Nq && pos >= 0 && pos < A.Lout) ob[co * A.Lout + pos] = A.bias ? v + bias : v;
      }
    }
}

// The same GEMM over rearranged weights with three K-steps of loads in
// flight: step kt issues the loads of step kt + 3 into the register slot
// that step kt's data has just left, computes step kt from LDS, then moves
// step kt + 1's registers into the other LDS buffer.  With one step of
// prefetch each of the 48 K-steps of Conv1d 512->512 k3 waited a whole
// memory round trip (about one wave per SIMD to cover it).  Buffer loads
// return zeros past the weight rows and, with the offset pushed out of
// range, at padding and past the output positions, so every step issues
// the same loads and the wait counts are exact; the last steps re-load
// the final K-step (unused).  Needs M Kg 2 and Cin L 4 below 2^31.
template <class T>
__global__ void __launch_bounds__(kThreads) convh_ring_kernel(HArgs A) {
  __shared__ __align__(16) _Float16 As[2][T::BM * kPitch];
  __shared__ __align__(16) _Float16 Bh[2][T::BN * kPitch];
  __shared__ __align__(16) _Float16 Bl[2][T::BN * kPitch];
  constexpr int WM_T = T::WM_T, WN_T = T::WN_T, BP = T::B_PAIRS;
  // A: a step's BM x 32 weight tile is BM * 4 16-byte pieces in a row;
  // thread t takes pieces t and t + 256 (as many as there are)
  constexpr int NPC = T::BM * 4, APT = (NPC + kThreads - 1) / kThreads;
  const unsigned mbits = *A.xmax;
  if (mbits >= 0x7f800000u) {  // an infinite or NaN activation: the fp32 kernels compute it
    if (threadIdx.x == 0) *A.flag = 1;  // every writer stores the same 1
    return;
  }
  const int kexp = convh_scale_exp(mbits);
  const float xscale = ldexpf(1.0f, kexp), unscale = ldexpf(1.0f, -kexp);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m_w = (wave / T::WAVES_N) * 32 * WM_T, n_w = (wave % T::WAVES_N) * 32 * WN_T;
  const uint3 tile = xcd_tile();  // neighbouring time tiles on one XCD
  const int64_t n0 = static_cast<int64_t>(tile.x) * T::BN;
  const int64_t m0 = static_cast<int64_t>(tile.y) * T::BM;
  const int64_t b = tile.z / A.ksplit;
  const int split = static_cast<int>(tile.z - b * A.ksplit);
  const int nk_all = static_cast<int>(A.Kg / kBK);
  const int kt0 = static_cast<int>(static_cast<int64_t>(nk_all) * split / A.ksplit);
  const int nk = static_cast<int>(static_cast<int64_t>(nk_all) * (split + 1) / A.ksplit) - kt0;
  const int Cin = static_cast<int>(A.Cin), L = static_cast<int>(A.L);
  const auto wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(A.wt), 0,
                                                     static_cast<int>(A.Kg * A.Mp * 2), 0x00020000);
  const auto xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(A.x + b * A.Cin * A.L), 0,
                                                     static_cast<int>(A.Cin * A.L * 4), 0x00020000);
  const int bn = tid % T::BN;
  const int64_t q = n0 + bn;
  const int q_pos = static_cast<int>(q * A.qs + A.tap_add);
  const bool q_in = q < A.Nq;
  struct Slot {
    uint4 a[APT];
    float b[BP][2];
  };
  Slot ring[3];
  // the next K-step to fetch (k0, its tap t and first channel ci0), moved
  // on after each fetch and held at the split's last step (the final
  // fetches repeat it): no division per step
  int f_k0 = kt0 * kBK, f_t = f_k0 / Cin, f_ci0 = f_k0 - f_t * Cin;
  const int k_last = (kt0 + nk - 1) * kBK;
  auto fetch = [&](Slot& sl) {
    const int k0 = f_k0, t = f_t, ci0 = f_ci0;
    if (f_k0 < k_last) {
      f_k0 += kBK;
      f_ci0 += kBK;
      if (f_ci0 >= Cin) {
        f_ci0 -= Cin;
        ++f_t;
      }
    }
    // the step's weight tile: Wt rows m0 .. m0+BM-1 of step k0 / 32, one
    // contiguous stretch (the old row-major Wt gave every lane of a load its
    // own cache line)
    const uint32_t ao = static_cast<uint32_t>(((k0 / kBK) * A.Mp + m0) * 64);
#pragma unroll
    for (int e = 0; e < APT; ++e) {
      const int pc = tid + kThreads * e;
      uint32_t off = pc < NPC ? ao + 16u * pc : 0x80000000u;
      asm volatile("" : "+v"(off));
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 0);
      sl.a[e] = make_uint4(v[0], v[1], v[2], v[3]);
    }
    const int pos = q_pos + t * static_cast<int>(A.tap_mul);
    const bool in = q_in && pos >= 0 && pos < L;
#pragma unroll
    for (int j = 0; j < BP; ++j) {
      const int kp = tid / T::BN + j * T::KP_STEP;
      uint32_t off = in ? static_cast<uint32_t>((ci0 + 2 * kp) * L + pos) * 4u : 0x80000000u;
      // the offset held in a register: without it the compiler turned the
      // select into a branch around each load, and the waits then covered
      // every load in flight
      asm volatile("" : "+v"(off));
      sl.b[j][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xrs, off, 0, 0));
      // (past the buffer stays past it: its size is below 2^31)
      sl.b[j][1] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xrs, off + 4u * L, 0, 0));
    }
  };
  auto stash = [&](const Slot& sl, int buf) {
#pragma unroll
    for (int e = 0; e < APT; ++e) {
      const int pc = tid + kThreads * e;  // row pc / 4, halves 8 (pc % 4)
      if (pc < NPC) *reinterpret_cast<uint4*>(&As[buf][(pc >> 2) * kPitch + 8 * (pc & 3)]) = sl.a[e];
    }
#pragma unroll
    for (int j = 0; j < BP; ++j) {
      const int kp = tid / T::BN + j * T::KP_STEP;
      h2 hi, lo;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float v = sl.b[j][e] * xscale;  // |v| < 2^15: exact
        const _Float16 h = static_cast<_Float16>(v);
        hi[e] = h;
        lo[e] = static_cast<_Float16>(v - static_cast<float>(h));
      }
      *reinterpret_cast<h2*>(&Bh[buf][bn * kPitch + 2 * kp]) = hi;
      *reinterpret_cast<h2*>(&Bl[buf][bn * kPitch + 2 * kp]) = lo;
    }
  };

  f16v acc[WM_T][WN_T];
#pragma unroll
  for (int i = 0; i < WM_T; ++i)
#pragma unroll
    for (int j = 0; j < WN_T; ++j)
#pragma unroll
      for (int g = 0; g < 16; ++g) acc[i][j][g] = 0.0f;

  fetch(ring[0]);
  fetch(ring[1]);
  fetch(ring[2]);
  stash(ring[0], 0);
  __syncthreads();
  auto step = [&](auto sc, int kt) {
    constexpr int S = decltype(sc)::value;  // kt % 3
    fetch(ring[S]);  // step min(kt + 3, nk - 1)
    const int buf = kt & 1;
#pragma unroll
    for (int ks = 0; ks < kBK; ks += 16) {
      const int kofs = ks + 8 * (lane >> 5);
      h8 a[WM_T], bh[WN_T], bl[WN_T];
#pragma unroll
      for (int i = 0; i < WM_T; ++i)
        a[i] = *reinterpret_cast<const h8*>(&As[buf][(m_w + 32 * i + (lane & 31)) * kPitch + kofs]);
#pragma unroll
      for (int j = 0; j < WN_T; ++j) {
        bh[j] = *reinterpret_cast<const h8*>(&Bh[buf][(n_w + 32 * j + (lane & 31)) * kPitch + kofs]);
        bl[j] = *reinterpret_cast<const h8*>(&Bl[buf][(n_w + 32 * j + (lane & 31)) * kPitch + kofs]);
      }
#pragma unroll
      for (int i = 0; i < WM_T; ++i)
#pragma unroll
        for (int j = 0; j < WN_T; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bh[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bl[j], acc[i][j], 0, 0, 0);
        }
    }
    if (kt + 1 < nk) stash(ring[(S + 1) % 3], buf ^ 1);
    __syncthreads();
  };
  // whole rounds of three steps, then the rest: an early exit between the
  // steps of a round put a wait for every load at the loop's head
  const int nr = nk / 3;
  for (int r = 0; r < nr; ++r) {
    step(std::integral_constant<int, 0>{}, 3 * r);
    step(std::integral_constant<int, 1>{}, 3 * r + 1);
    step(std::integral_constant<int, 2>{}, 3 * r + 2);
  }
  if (3 * nr < nk) step(std::integral_constant<int, 0>{}, 3 * nr);
  if (3 * nr + 1 < nk) step(std::integral_constant<int, 1>{}, 3 * nr + 1);

  // D(i, j) of a 32x32 tile: lane j + 32 * ((i / 4) % 2), register (i / 8) * 4 + i % 4
  if (A.part) {  // this split's raw sums
    float* pb = A.part + (b * A.ksplit + split) * A.M * A.Nq;
#pragma unroll
    for (int i = 0; i < WM_T; ++i)
#pragma unroll
      for (int g = 0; g < 16; ++g) {
        const int64_t m = m0 + m_w + 32 * i + 8 * (g / 4) + 4 * (lane >> 5) + (g % 4);
        if (m >= A.M) continue;
#pragma unroll
        for (int j = 0; j < WN_T; ++j) {
          const int64_t qq = n0 + n_w + 32 * j + (lane & 31);
          if (qq < A.Nq) pb[m * A.Nq + qq] = acc[i][j][g];
        }
      }
    return;
  }
  float* ob = A.out + b * A.Cout * A.Lout;
#pragma unroll
  for (int i = 0; i < WM_T; ++i)
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      const int64_t m = m0 + m_w + 32 * i + 8 * (g / 4) + 4 * (lane >> 5) + (g % 4);
      if (m >= A.M) continue;
      const int64_t co = m / A.P, r = m - co * A.P;
      const float bias = A.bias ? A.bias[co] : 0.0f;
      const float sc = A.dq.scale ? load_as_f32(A.dq.scale, A.dq.scale_dt, co * A.dq.scale_stride)
                                  : 1.0f;
#pragma unroll
      for (int j = 0; j < WN_T; ++j) {
        const int64_t qq = n0 + n_w + 32 * j + (lane & 31);
        const float u = acc[i][j][g] * unscale;  // exact: a power of two
        const float v = A.dq.scale ? u * sc : u;
        const int64_t pos = qq * A.os + r + A.ophase0;
        if (qq < A.Nq && pos >= 0 && pos < A.Lout) ob[co * A.Lout + pos] = A.bias ? v + bias : v;
      }
    }
}

// Split-K's finish: out[b, co, pos] = the splits' sums at (m, q) added in
// split order, then the epilogue above, where pos - ophase0 = q P + r and
// m = co P + r (P = os: one phase per output position).  A thread per
// output position (blocks along the row on x, channels on y, batch on z),
// so the stores run along each output row; 32-bit indexes (the host keeps
// M Nq and Cout Lout below 2^31).  Nothing to do after a non-finite
// activation (the fp32 kernels compute the convolution).
__global__ void __launch_bounds__(256) convh_splitk_finish(HArgs A) {
  const unsigned mbits = *A.xmax;
  if (mbits >= 0x7f800000u) return;
  const float unscale = ldexpf(1.0f, -convh_scale_exp(mbits));
  const int P = A.P, Nq = static_cast<int>(A.Nq), Lout = static_cast<int>(A.Lout);
  const int MN = static_cast<int>(A.M * A.Nq), ks = A.ksplit, ph0 = static_cast<int>(A.ophase0);
  const int b = blockIdx.z;
  for (int co = blockIdx.y; co < static_cast<int>(A.Cout); co += gridDim.y) {
    const float bias = A.bias ? A.bias[co] : 0.0f;
    const float sc = A.dq.scale ? load_as_f32(A.dq.scale, A.dq.scale_dt, co * A.dq.scale_stride)
                                : 1.0f;
    const float* pb = A.part + static_cast<int64_t>(b) * ks * MN;
    float* orow = A.out + (static_cast<int64_t>(b) * A.Cout + co) * Lout;
    for (int pos = blockIdx.x * blockDim.x + threadIdx.x; pos < Lout; pos += gridDim.x * blockDim.x) {
      const int u = pos - ph0;
      if (u < 0) continue;
      const int q = u / P, r = u - q * P;
      if (q >= Nq) continue;
      const int i = (co * P + r) * Nq + q;
      float acc = pb[i];
      for (int sp = 1; sp < ks; ++sp) acc += pb[sp * MN + i];
      const float v0 = acc * unscale;  // exact: a power of two
      const float v = A.dq.scale ? v0 * sc : v0;
      orow[pos] = A.bias ? v + bias : v;
    }
  }
}

__global__ void convh_flag_clear(int* flag, unsigned* xmax) {
  *flag = 0;
  *xmax = 0u;
}

// *xmax = max(*xmax, bits of max |x|) over n floats: |x| is a non-negative
// float (NaN above infinity), so its bits order as unsigned integers.
// vec: x is 16-byte aligned.
__global__ void __launch_bounds__(256) convh_absmax(const float* __restrict__ x, int64_t n, int vec,
                                                    unsigned* xmax) {
  __shared__ unsigned part[4];
  unsigned m = 0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t t0 = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  int64_t done = 0;
  if (vec) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const int64_t n4 = n / 4;
    for (int64_t i = t0; i < n4; i += stride) {
      const float4 v = x4[i];
      m = max(m, max(max(__float_as_uint(fabsf(v.x)), __float_as_uint(fabsf(v.y))),
                     max(__float_as_uint(fabsf(v.z)), __float_as_uint(fabsf(v.w)))));
    }
    done = 4 * n4;
  }
  for (int64_t i = done + t0; i < n; i += stride) m = max(m, __float_as_uint(fabsf(x[i])));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = max(m, static_cast<unsigned>(__shfl_xor(static_cast<int>(m), off, 64)));
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) atomicMax(xmax, max(max(part[0], part[1]), max(part[2], part[3])));
}

// Wt[kk / 32][m][kk % 32] (m = co*P + r, kk = t*Cin + ci; Mp rows a step,
// zeros past M): the fp16 value the gathering kernel forms, W less the zero
// point (0 past the kernel for transposed), stored step by step so that a
// step's weight tile is one stretch.
// Rows m on the grid's y axis, kk along x, 32-bit index arithmetic (the
// host checks the weight count and M * Kg against 2^31): a flat 64-bit walk
// with a division chain per element took 16.8 us for ConvTranspose1d
// 512->256 k20's 2.6M values, this 14 us -- bound by the transposed
// weights' reads, one cache line per element (a block per output channel
// staging its weights through LDS measured slower, 23 us).
template <typename TW>
__global__ void __launch_bounds__(256) convh_weights(_Float16* __restrict__ wt, HArgs A) {
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
    *A.flag = 0;
    *A.xmax = 0u;
  }
  const TW* w = static_cast<const TW*>(A.w);
  const int P = A.P, Kg = static_cast<int>(A.Kg), Cin = static_cast<int>(A.Cin);
  const int Kw = static_cast<int>(A.Kw), s = static_cast<int>(A.s);
  const int M = static_cast<int>(A.M), Mp = static_cast<int>(A.Mp), cout = M / P;
  for (int m = blockIdx.y; m < Mp; m += gridDim.y) {
    const int co = m / P, r = m - co * P;
    const float zp = A.dq.zp && m < M ? load_as_f32(A.dq.zp, A.dq.zp_dt, co * A.dq.zp_stride) : 0.0f;
    for (int kk = blockIdx.x * blockDim.x + threadIdx.x; kk < Kg; kk += gridDim.x * blockDim.x) {
      const int t = kk / Cin, ci = kk - t * Cin;
      const int tap = A.transposed ? r + s * t : t;
      float v = 0.0f;
      if (m < M && tap < Kw) {
        const int idx = A.transposed ? (ci * cout + co) * Kw + tap : (co * Cin + ci) * Kw + tap;
        v = static_cast<float>(w[idx]) - zp;
      }
      wt[(static_cast<int64_t>(kk / kBK) * Mp + m) * kBK + (kk % kBK)] = static_cast<_Float16>(v);
    }
  }
}

// The ring kernel's 32-bit buffer offsets: weights (step-major) and one
// batch of activations below 2^31 bytes; else the gathering kernel runs.
static bool ring_ok(const HArgs& a) {
  return a.Kg * a.Mp * 2 < (int64_t{1} << 31) && a.Cin * a.L * 4 < (int64_t{1} << 31);
}

// Rearranged weights (a.wt) go to the ring kernel, else the kernel gathers
// them from W.
template <class T, typename TW>
static void launch_t(const HArgs& a, const dim3& grid) {
  if (a.wt)
    KK_LAUNCH((convh_ring_kernel<T>), grid, dim3(kThreads), 0, ctx().stream, a);
  else
    KK_LAUNCH((convh_kernel<T, TW, false>), grid, dim3(kThreads), 0, ctx().stream, a);
}

// Split-K count for the ring kernel: enough splits that every CU gets two
// blocks, at most 4, at least 8 K-steps a split, and the partial sums
// within `part_bytes` (the context scratch left beside the rearranged
// weights); 1 when no CU is short.  The choice depends on sizes alone, so a
// call recorded into a graph sums in the same order as the same call made
// eagerly.
template <class T>
static int ksplit_for(const HArgs& a, int64_t batch, size_t part_bytes) {
  const int64_t cus = ctx().num_cus > 0 ? ctx().num_cus : 256;
  const int64_t blocks = batch * ceil_div(a.Nq, T::BN) * ceil_div(a.M, T::BM);
  if (!a.wt || blocks >= 2 * cus || a.M * a.Nq >= (int64_t{1} << 31) / 4 ||
      a.Cout * a.Lout >= (int64_t{1} << 31))
    return 1;
  const int64_t nk = a.Kg / kBK;
  const int64_t room = static_cast<int64_t>(part_bytes) / (4 * batch * a.M * a.Nq);
  const int64_t s = std::min<int64_t>({4, ceil_div(2 * cus, blocks), nk / 8, room});
  return static_cast<int>(std::max<int64_t>(1, s));
}

template <class T>
static void launch(HArgs& a, int w_dt, int64_t batch, float* part, size_t part_bytes) {
  a.ksplit = ksplit_for<T>(a, batch, part_bytes);
  a.part = a.ksplit > 1 ? part : nullptr;
  const dim3 grid(static_cast<unsigned>(ceil_div(a.Nq, T::BN)), static_cast<unsigned>(ceil_div(a.M, T::BM)),
                  static_cast<unsigned>(batch * a.ksplit));
  if (w_dt == KK_F16) launch_t<T, _Float16>(a, grid);
  else if (w_dt == KK_I8) launch_t<T, int8_t>(a, grid);
  else launch_t<T, uint8_t>(a, grid);
  if (a.part) {
    const dim3 fg(static_cast<unsigned>(std::min<int64_t>(ceil_div(a.Lout, 256), 64)),
                  static_cast<unsigned>(std::min<int64_t>(a.Cout, 65535)), static_cast<unsigned>(batch));
    KK_LAUNCH(convh_splitk_finish, fg, dim3(256), 0, ctx().stream, a);
    a.part = nullptr;
    a.ksplit = 1;
  }
}

// Rearranges the weights into the context scratch (or, larger, into a
// pooled workspace unless a graph is being recorded; else the kernel
// gathers them); launches the tile that suits M x Nq.
static void run(HArgs& a, const kk_tensor* w, int64_t batch, void** ws) {
  a.Mp = ceil_div(a.M, 128) * 128;
  const size_t wt_bytes = static_cast<size_t>(a.Kg * a.Mp * 2);
  void* wtp = nullptr;
  if (!ring_ok(a)) wtp = nullptr;
  else if (wt_bytes <= kScratchBytes) wtp = ctx().scratch;
  else if (!ctx().capturing && kk_alloc(wt_bytes, ws) == KK_OK) wtp = *ws;
  if (wtp) {
    _Float16* wt = static_cast<_Float16*>(wtp);
    const dim3 g(static_cast<unsigned>(std::min<int64_t>(ceil_div(a.Kg, 256), 64)),
                 static_cast<unsigned>(std::min<int64_t>(a.Mp, 65535)));
    if (w->dtype == KK_F16)
      KK_LAUNCH(convh_weights<_Float16>, g, dim3(256), 0, ctx().stream, wt, a);
    else if (w->dtype == KK_I8)
      KK_LAUNCH(convh_weights<int8_t>, g, dim3(256), 0, ctx().stream, wt, a);
    else
      KK_LAUNCH(convh_weights<uint8_t>, g, dim3(256), 0, ctx().stream, wt, a);
    a.wt = wt;
  } else {
    KK_LAUNCH(convh_flag_clear, dim3(1), dim3(1), 0, ctx().stream, a.flag, a.xmax);
  }
  {
    const int64_t n = a.Cin * a.L * batch;
    const unsigned g = static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 256 * 16), 1024)));
    const int vec = reinterpret_cast<uintptr_t>(a.x) % 16 == 0 ? 1 : 0;
    KK_LAUNCH(convh_absmax, dim3(g), dim3(256), 0, ctx().stream, a.x, n, vec, a.xmax);
  }
  // split-K partial sums: the context scratch beside weights rearranged there
  float* part = nullptr;
  size_t part_bytes = 0;
  if (wtp == ctx().scratch) {
    const size_t off = (wt_bytes + 255) & ~size_t{255};
    if (off < kScratchBytes) {
      part = reinterpret_cast<float*>(static_cast<char*>(ctx().scratch) + off);
      part_bytes = kScratchBytes - off;
    }
  }
  // the largest tile that still gives every CU two blocks; 128 x 32 below that
  const int64_t cus = ctx().num_cus > 0 ? ctx().num_cus : 256;
  if (a.M <= 32) launch<Tile<1, 1, 1>>(a, w->dtype, batch, part, part_bytes);
  else if (a.M <= 64) launch<Tile<2, 1, 2>>(a, w->dtype, batch, part, part_bytes);
  else if (batch * ceil_div(a.M, 128) * ceil_div(a.Nq, 128) >= 2 * cus)
    launch<Tile<2, 2, 2>>(a, w->dtype, batch, part, part_bytes);
  else launch<Tile<4, 1, 1>>(a, w->dtype, batch, part, part_bytes);
}

}  // namespace convh

using namespace convh;

// Launches the fp16 matrix-core convolution when it applies and returns
// true; *flag is then the condition for the caller's fp32 fallback, which
// the caller launches next, and *ws a workspace to kk_free after that (or
// NULL).  The flag is cleared at the start of each call (by the weight
// rearrangement, or a one-thread kernel when there is none).
bool convh_run(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w, const Dequant& dq,
               const kk_tensor* bias, bool transposed, int64_t stride, int64_t dilation,
               int64_t pad0, int64_t Nq, int** flag, void** ws) {
  *ws = nullptr;
  // fp16 weights as they are; 8-bit weights less an 8-bit zero point
  const bool w16 = w->dtype == KK_F16 && !dq.active;
  const bool w8 = (w->dtype == KK_I8 || w->dtype == KK_U8) &&
                  (!dq.zp || dq.zp_dt == KK_I8 || dq.zp_dt == KK_U8);
  if (!(w16 || w8) || x->dtype != KK_F32) return false;
  const int64_t N = x->shape[0], Cin = x->shape[1], L = x->shape[2];
  const int64_t Cout = out->shape[1], Lout = out->shape[2], Kw = w->shape[2];
  if (Cin % kBK || (transposed && dilation != 1)) return false;
  const int64_t taps = transposed ? ceil_div(Kw, stride) : Kw;
  const int64_t P = transposed ? stride : 1;
  const int64_t Kg = taps * Cin, M = P * Cout;
  if (M * Nq * Kg < (int64_t{1} << 26) || N > 65535 || ceil_div(M, 32) > 65535 ||
      ceil_div(Nq, 32) > 0x7fffffff || numel(w) > 0x7fffffff)
    return false;
  *flag = ctx().row_counters + kRowCounters + kFlagConvh;
  HArgs a{};
  a.w = w->data; a.transposed = transposed ? 1 : 0; a.Kw = Kw; a.s = stride; a.dq = dq;
  a.x = static_cast<const float*>(x->data); a.out = static_cast<float*>(out->data);
  a.bias = bias ? static_cast<const float*>(bias->data) : nullptr; a.flag = *flag;
  a.xmax = reinterpret_cast<unsigned*>(ctx().row_counters + kRowCounters + kFlagConvhMax);
  a.Cin = Cin; a.L = L; a.M = M; a.Cout = Cout; a.Kg = Kg; a.Nq = Nq; a.Lout = Lout;
  a.P = static_cast<int>(P);
  a.ksplit = 1;
  if (transposed) {
    a.qs = 1; a.tap_mul = -1; a.tap_add = 0; a.os = stride; a.ophase0 = -pad0;
  } else {
    a.qs = stride; a.tap_mul = dilation; a.tap_add = -pad0; a.os = 1; a.ophase0 = 0;
  }
  run(a, w, N, ws);
  return true;
}


}  // namespace kk
