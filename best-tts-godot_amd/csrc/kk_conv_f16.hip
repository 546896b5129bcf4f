// Conv1d and ConvTranspose1d with fp16 weights on the fp16 matrix cores,
// fp32 results.
//
// An fp16 weight is exact in fp16.  Each fp32 activation x is split into
// hi = fp16(x) and lo = fp16(x - hi) (x - hi is exact in fp32), so hi + lo
// equals x to within 2^-22 |x|; every product w*hi and w*lo is exact in
// fp32 (11 + 11 significant bits), and v_mfma_f32_32x32x16_f16 accumulates
// them in fp32: the accuracy of fp32 products accumulated in fp32, at the
// fp16 matrix rate.  An activation of magnitude >= 2^15 (fp16 ends at
// 65504) or infinite sets a flag instead; the fp32 kernels, launched after
// this one with that flag as their condition, then redo the convolution.
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
// The weights are rearranged into Wt by a small kernel in the same call.
#include <algorithm>

#include "kk_internal.h"

namespace kk {
namespace convh {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int kBK = 32;        // K-step (halves)
constexpr int kPitch = kBK + 8;  // LDS row pitch (halves): 80 bytes
constexpr int kThreads = 256;

struct HArgs {
  const _Float16* wt;  // [M = Cout*P][Kg]
  const float* x;      // [N, Cin, L]
  float* out;          // [N, Cout, Lout]
  const float* bias;   // [Cout] or NULL
  int* flag;
  int64_t Cin, L, M, Cout, Kg, Nq, Lout;
  int64_t qs, tap_mul, tap_add, os, ophase0;
  int P;
};

// WAVES_M x (4 / WAVES_M) wavefronts, each owning WM_T x WN_T tiles of 32x32.
template <int WAVES_M_, int WM_T_, int WN_T_>
struct Tile {
  static constexpr int WAVES_M = WAVES_M_, WM_T = WM_T_, WN_T = WN_T_;
  static constexpr int WAVES_N = 4 / WAVES_M;
  static constexpr int BM = WAVES_M * 32 * WM_T, BN = WAVES_N * 32 * WN_T;
  // A staging: BM rows of 4 chunks of 8 halves
  static constexpr int A_CHUNKS = BM * 4;
  static constexpr int A_PER = (A_CHUNKS + kThreads - 1) / kThreads;
  // B staging: thread -> column n = t % BN, k pairs t / BN + j * (256 / BN)
  static constexpr int KP_STEP = kThreads / BN;
  static constexpr int B_PAIRS = (kBK / 2) / KP_STEP;
  static_assert(kThreads % BN == 0 && (kBK / 2) % KP_STEP == 0, "B staging shape");
};

template <class T>
__global__ void __launch_bounds__(kThreads) convh_kernel(HArgs A) {
  __shared__ __align__(16) _Float16 As[2][T::BM * kPitch];
  __shared__ __align__(16) _Float16 Bh[2][T::BN * kPitch];
  __shared__ __align__(16) _Float16 Bl[2][T::BN * kPitch];
  constexpr int WM_T = T::WM_T, WN_T = T::WN_T;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m_w = (wave / T::WAVES_N) * 32 * WM_T, n_w = (wave % T::WAVES_N) * 32 * WN_T;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * T::BN;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * T::BM;
  const int64_t b = blockIdx.z;
  const _Float16* wt = A.wt;
  const float* xb = A.x + b * A.Cin * A.L;
  const int64_t nk = A.Kg / kBK;

  // staging registers
  uint4 areg[T::A_PER];
  float bv[T::B_PAIRS][2];
  bool bad = false;
  const int bn = tid % T::BN;
  const int64_t q = n0 + bn;
  auto fetch = [&](int64_t k0) {
#pragma unroll
    for (int p = 0; p < T::A_PER; ++p) {
      const int c = tid + p * kThreads;
      areg[p] = make_uint4(0, 0, 0, 0);
      if (c < T::A_CHUNKS) {
        const int64_t row = m0 + c / 4;
        if (row < A.M)
          areg[p] = *reinterpret_cast<const uint4*>(wt + row * A.Kg + k0 + 8 * (c % 4));
      }
    }
    const int64_t t = k0 / A.Cin, ci0 = k0 - t * A.Cin;
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
    for (int p = 0; p < T::A_PER; ++p) {
      const int c = tid + p * kThreads;
      if (c < T::A_CHUNKS)
        *reinterpret_cast<uint4*>(&As[buf][(c / 4) * kPitch + 8 * (c % 4)]) = areg[p];
    }
#pragma unroll
    for (int j = 0; j < T::B_PAIRS; ++j) {
      const int kp = tid / T::BN + j * T::KP_STEP;
      h2 hi, lo;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float v = bv[j][e];
        bad |= !(fabsf(v) < 32768.0f) && !(v != v);  // too large, or infinite (NaN passes)
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
  if (bad) *A.flag = 1;  // every writer stores the same 1

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
#pragma unroll
      for (int j = 0; j < WN_T; ++j) {
        const int64_t qq = n0 + n_w + 32 * j + (lane & 31);
        const int64_t pos = qq * A.os + r + A.ophase0;
        if (qq < A.Nq && pos >= 0 && pos < A.Lout)
          ob[co * A.Lout + pos] = A.bias ? acc[i][j][g] + bias : acc[i][j][g];
      }
    }
}

// Wt from W (fp16): conv (transposed = 0) W [Cout][Cin][K] -> Wt[co][k*Cin + ci];
// transposed W [Cin][Cout][K] -> Wt[co*P + r][m*Cin + ci] = W[ci][co][r + s*m].
// Also clears the overflow flag.
__global__ void convh_weights(_Float16* __restrict__ wt, const _Float16* __restrict__ w,
                              int64_t Cout, int64_t Cin, int64_t Kw, int64_t taps, int64_t P,
                              int64_t s, int transposed, int* flag) {
  const int64_t Kg = taps * Cin, total = P * Cout * Kg;
  if (blockIdx.x == 0 && threadIdx.x == 0) *flag = 0;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t kk = i % Kg, m = i / Kg;
    const int64_t co = m / P, r = m - co * P;
    const int64_t t = kk / Cin, ci = kk % Cin;
    _Float16 v = static_cast<_Float16>(0.0f);
    if (!transposed) {
      v = w[(co * Cin + ci) * Kw + t];
    } else {
      const int64_t k = r + s * t;
      if (k < Kw) v = w[(ci * Cout + co) * Kw + k];
    }
    wt[i] = v;
  }
}

template <class T>
static void launch(const HArgs& a, int64_t batch) {
  const dim3 grid(static_cast<unsigned>(ceil_div(a.Nq, T::BN)), static_cast<unsigned>(ceil_div(a.M, T::BM)),
                  static_cast<unsigned>(batch));
  hipLaunchKernelGGL(convh_kernel<T>, grid, dim3(kThreads), 0, ctx().stream, a);
}

}  // namespace convh

using namespace convh;

// Launches the fp16-weight convolution when it applies and returns true;
// *flag then points at the overflow flag (in *ws, which the caller frees
// after launching its fp32 fallback with that flag as condition).
bool convh_run(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w, const kk_tensor* bias,
               bool transposed, int64_t stride, int64_t dilation, int64_t pad0, int64_t Nq,
               void** ws, int** flag, int* rc) {
  *rc = KK_OK;
  if (w->dtype != KK_F16 || x->dtype != KK_F32) return false;
  const int64_t N = x->shape[0], Cin = x->shape[1], L = x->shape[2];
  const int64_t Cout = out->shape[1], Lout = out->shape[2], Kw = w->shape[2];
  if (Cin % 32 || (transposed && dilation != 1)) return false;
  const int64_t taps = transposed ? ceil_div(Kw, stride) : Kw;
  const int64_t P = transposed ? stride : 1;
  const int64_t Kg = taps * Cin, M = P * Cout;
  if (M * Nq * Kg < (int64_t{1} << 27) || N > 65535 || ceil_div(M, 32) > 65535 ||
      ceil_div(Nq, 128) > 0x7fffffff)
    return false;
  const int64_t wt_bytes = ceil_div(M * Kg * 2, 256) * 256;
  *rc = kk_alloc(static_cast<size_t>(wt_bytes + 256), ws);
  if (*rc != KK_OK) return false;
  _Float16* wt = static_cast<_Float16*>(*ws);
  *flag = reinterpret_cast<int*>(static_cast<char*>(*ws) + wt_bytes);
  const int64_t total = M * Kg;
  hipLaunchKernelGGL(convh_weights, dim3(static_cast<unsigned>(std::min<int64_t>(ceil_div(total, 256), 4096))),
                     dim3(256), 0, ctx().stream, wt, static_cast<const _Float16*>(w->data), Cout, Cin,
                     Kw, taps, P, stride, transposed ? 1 : 0, *flag);
  HArgs a{};
  a.wt = wt; a.x = static_cast<const float*>(x->data); a.out = static_cast<float*>(out->data);
  a.bias = bias ? static_cast<const float*>(bias->data) : nullptr; a.flag = *flag;
  a.Cin = Cin; a.L = L; a.M = M; a.Cout = Cout; a.Kg = Kg; a.Nq = Nq; a.Lout = Lout;
  a.P = static_cast<int>(P);
  if (transposed) {
    a.qs = 1; a.tap_mul = -1; a.tap_add = 0; a.os = stride; a.ophase0 = -pad0;
  } else {
    a.qs = stride; a.tap_mul = dilation; a.tap_add = -pad0; a.os = 1; a.ophase0 = 0;
  }
  if (M <= 32) launch<Tile<1, 1, 1>>(a, N);
  else if (M <= 64) launch<Tile<2, 1, 2>>(a, N);
  else launch<Tile<2, 2, 2>>(a, N);
  *rc = check_launch("convh_kernel");
  return true;
}

}  // namespace kk
