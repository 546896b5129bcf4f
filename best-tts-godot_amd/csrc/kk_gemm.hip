// Contractions: batched MatMul with weight dequantisation, Conv1d as an
// implicit GEMM and ConvTranspose1d as a phase-decomposed implicit GEMM, all
// on one fp32 MFMA core (v_mfma_f32_16x16x4_f32: fp32 operands, exact fp32
// products, fp32 accumulation -- the fp32 semantics of the numpy reference).
//
// Core: a block of four wavefronts computes a BM x BN tile of C = A . B in
// K-steps of 32.  Each wavefront owns a (16*WTM) x (16*WTN) sub-tile made of
// WTM x WTN MFMA 16x16 tiles.  Tile loaders -- vectorised dense loaders for
// fp32 activations and int8/uint8/fp16/fp32 weights, an im2col gather for
// the convolution input, scalar gathers for everything else -- fetch the
// next K-step from global memory into registers while the current one is
// multiplied, dequantise there ((q - zp) * scale in fp32, with the scale and
// zero point held in registers), and store it K-major in LDS.
#include <algorithm>
#include <type_traits>

#include "kk_internal.h"

namespace kk {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kBK = 32;   // K-step
constexpr int kPad = 4;   // LDS row padding (floats)
constexpr int kNT = 256;  // threads per block (4 wavefronts)

template <int BM_, int BN_, int WTM_, int WTN_>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, WTM = WTM_, WTN = WTN_;
  static constexpr int WM = 16 * WTM, WN = 16 * WTN;
  static constexpr int WAVES_N = BN / WN;
  static constexpr int PA = BM + kPad, PB = BN + kPad;
  static_assert((BM / WM) * (BN / WN) == 4, "four wavefronts per block");
};
using CfgL = Cfg<64, 64, 2, 2>;  // 32x32 per wave
using CfgM = Cfg<64, 32, 1, 2>;  // 16x32 per wave
using CfgS = Cfg<32, 32, 1, 1>;  // 16x16 per wave

// Scale and zero point of one weight row/column, read once per block.
// A NULL scale means 1 (the integer ops shift by their zero point only).
__device__ __forceinline__ void dq_params(const Dequant& dq, int64_t idx, float& s, float& z) {
  s = dq.scale ? load_as_f32(dq.scale, dq.scale_dt, idx * dq.scale_stride) : 1.0f;
  z = dq.zp ? load_as_f32(dq.zp, dq.zp_dt, idx * dq.zp_stride) : 0.0f;
}

// Four consecutive elements of type T starting at p (4-element aligned).
template <typename T>
__device__ __forceinline__ float4 load4(const T* p);
template <>
__device__ __forceinline__ float4 load4<float>(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}
template <>
__device__ __forceinline__ float4 load4<__half>(const __half* p) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  const __half2 lo = *reinterpret_cast<const __half2*>(&u.x);
  const __half2 hi = *reinterpret_cast<const __half2*>(&u.y);
  return make_float4(__low2float(lo), __high2float(lo), __low2float(hi), __high2float(hi));
}
template <>
__device__ __forceinline__ float4 load4<int8_t>(const int8_t* p) {
  const uint32_t u = *reinterpret_cast<const uint32_t*>(p);
  return make_float4(static_cast<float>(static_cast<int8_t>(u & 0xff)),
                     static_cast<float>(static_cast<int8_t>((u >> 8) & 0xff)),
                     static_cast<float>(static_cast<int8_t>((u >> 16) & 0xff)),
                     static_cast<float>(static_cast<int8_t>(u >> 24)));
}
template <>
__device__ __forceinline__ float4 load4<uint8_t>(const uint8_t* p) {
  const uint32_t u = *reinterpret_cast<const uint32_t*>(p);
  return make_float4(static_cast<float>(u & 0xff), static_cast<float>((u >> 8) & 0xff),
                     static_cast<float>((u >> 16) & 0xff), static_cast<float>(u >> 24));
}

template <typename T>
constexpr bool is_quant() {
  return std::is_same<T, int8_t>::value || std::is_same<T, uint8_t>::value;
}

// ---------------------------------------------------------------- loaders
// A loaders fill As[k][m] (pitch PA), B loaders fill Bs[k][n] (pitch PB).
// fetch(k0) reads the K-step starting at k0 into registers; stash() writes
// them to LDS.  Out-of-range elements are zero.

// A [M, K] with K contiguous, element type T, optional per-row (or
// per-tensor) dequantisation; needs K % 4 == 0 and 4-element-aligned rows.
template <class C, typename T>
struct AQuad {
  static constexpr int QPR = kBK / 4;
  static constexpr int RPP = kNT / QPR;
  static constexpr int P = (C::BM + RPP - 1) / RPP;
  const T* ptr[P];
  bool ok[P];
  float s[P], z[P];
  float4 v[P];
  int kq, r0;
  int64_t K;
  __device__ __forceinline__ void init(const T* a, int64_t lda, int64_t M, int64_t K_, int64_t m0,
                                       const Dequant& dq) {
    kq = (threadIdx.x % QPR) * 4;
    r0 = threadIdx.x / QPR;
    K = K_;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int row = r0 + p * RPP;
      ok[p] = row < C::BM && m0 + row < M;
      ptr[p] = a + (ok[p] ? (m0 + row) * lda : 0);
      s[p] = 1.0f;
      z[p] = 0.0f;
      if (is_quant<T>() && ok[p]) dq_params(dq, m0 + row, s[p], z[p]);
    }
  }
  __device__ __forceinline__ void fetch(int64_t k0) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      if (ok[p] && k0 + kq < K) {
        float4 t = load4<T>(ptr[p] + k0 + kq);
        if (is_quant<T>()) {
          t.x = (t.x - z[p]) * s[p];
          t.y = (t.y - z[p]) * s[p];
          t.z = (t.z - z[p]) * s[p];
          t.w = (t.w - z[p]) * s[p];
        }
        v[p] = t;
      } else {
        v[p] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
  }
  __device__ __forceinline__ void stash(float* As) const {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int row = r0 + p * RPP;
      if (row < C::BM) {
        As[(kq + 0) * C::PA + row] = v[p].x;
        As[(kq + 1) * C::PA + row] = v[p].y;
        As[(kq + 2) * C::PA + row] = v[p].z;
        As[(kq + 3) * C::PA + row] = v[p].w;
      }
    }
  }
};

// B [K, N] with N contiguous, element type T, optional per-column (or
// per-tensor) dequantisation; needs N % 4 == 0 and 4-element-aligned rows.
template <class C, typename T>
struct BQuad {
  static constexpr int QPR = C::BN / 4;
  static constexpr int RPP = kNT / QPR;
  static constexpr int P = kBK / RPP;
  const T* base;
  int64_t ldb, K;
  bool col_ok;
  float s[4], z[4];
  float4 v[P];
  int nq, r0;
  __device__ __forceinline__ void init(const T* b, int64_t ldb_, int64_t N, int64_t K_, int64_t n0,
                                       const Dequant& dq) {
    nq = (threadIdx.x % QPR) * 4;
    r0 = threadIdx.x / QPR;
    ldb = ldb_;
    K = K_;
    col_ok = n0 + nq < N;
    base = b + (col_ok ? n0 + nq : 0);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      s[c] = 1.0f;
      z[c] = 0.0f;
      if (is_quant<T>() && col_ok) dq_params(dq, n0 + nq + c, s[c], z[c]);
    }
  }
  __device__ __forceinline__ void fetch(int64_t k0) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int64_t k = k0 + r0 + p * RPP;
      if (col_ok && k < K) {
        float4 t = load4<T>(base + k * ldb);
        if (is_quant<T>()) {
          t.x = (t.x - z[0]) * s[0];
          t.y = (t.y - z[1]) * s[1];
          t.z = (t.z - z[2]) * s[2];
          t.w = (t.w - z[3]) * s[3];
        }
        v[p] = t;
      } else {
        v[p] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
  }
  __device__ __forceinline__ void stash(float* Bs) const {
#pragma unroll
    for (int p = 0; p < P; ++p)
      *reinterpret_cast<float4*>(Bs + (r0 + p * RPP) * C::PB + nq) = v[p];
  }
};

// Scalar gathers through a functor get(i, j) (bounds-checked by the
// functor).  The FAST flag selects which tile dimension consecutive threads
// walk (the operand's unit-stride direction, for coalescing).
template <class C, class Get, bool KFAST>
struct AScalar {
  static constexpr int E = C::BM * kBK / kNT;
  Get get;
  int64_t m0;
  float v[E];
  __device__ __forceinline__ void idx(int e, int& m, int& k) const {
    if (KFAST) { m = e / kBK; k = e % kBK; } else { m = e % C::BM; k = e / C::BM; }
  }
  __device__ __forceinline__ void fetch(int64_t k0) {
#pragma unroll
    for (int t = 0; t < E; ++t) {
      int m, k;
      idx(threadIdx.x + t * kNT, m, k);
      v[t] = get(m0 + m, k0 + k);
    }
  }
  __device__ __forceinline__ void stash(float* As) const {
#pragma unroll
    for (int t = 0; t < E; ++t) {
      int m, k;
      idx(threadIdx.x + t * kNT, m, k);
      As[k * C::PA + m] = v[t];
    }
  }
};

template <class C, class Get, bool NFAST>
struct BScalar {
  static constexpr int E = kBK * C::BN / kNT;
  Get get;
  int64_t n0;
  float v[E];
  __device__ __forceinline__ void idx(int e, int& k, int& n) const {
    if (NFAST) { k = e / C::BN; n = e % C::BN; } else { n = e / kBK; k = e % kBK; }
  }
  __device__ __forceinline__ void fetch(int64_t k0) {
#pragma unroll
    for (int t = 0; t < E; ++t) {
      int k, n;
      idx(threadIdx.x + t * kNT, k, n);
      v[t] = get(k0 + k, n0 + n);
    }
  }
  __device__ __forceinline__ void stash(float* Bs) const {
#pragma unroll
    for (int t = 0; t < E; ++t) {
      int k, n;
      idx(threadIdx.x + t * kNT, k, n);
      Bs[k * C::PB + n] = v[t];
    }
  }
};

// Conv1d input as the B operand: B[kk, l] = x[ci, l*s + k*d - p0] with
// kk = ci*Kw + k; each thread gathers four consecutive l of one kk.
template <class C>
struct BIm2col {
  static constexpr int QPR = C::BN / 4;
  static constexpr int RPP = kNT / QPR;
  static constexpr int P = kBK / RPP;
  const float* x;  // this batch item's [Cin, L]
  int64_t L, Kw, s, d, p0, Kdim, Lout;
  int64_t l0;      // first output position of this thread's quad
  float4 v[P];
  int r0;
  __device__ __forceinline__ void fetch(int64_t k0) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int64_t kk = k0 + r0 + p * RPP;
      float e[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (kk < Kdim) {
        const int64_t ci = kk / Kw, k = kk - ci * Kw;
        const float* xr = x + ci * L;
        const int64_t pos0 = l0 * s + k * d - p0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int64_t pos = pos0 + c * s;
          if (l0 + c < Lout && pos >= 0 && pos < L) e[c] = xr[pos];
        }
      }
      v[p] = make_float4(e[0], e[1], e[2], e[3]);
    }
  }
  __device__ __forceinline__ void stash(float* Bs) const {
    const int nq = (threadIdx.x % QPR) * 4;
#pragma unroll
    for (int p = 0; p < P; ++p)
      *reinterpret_cast<float4*>(Bs + (r0 + p * RPP) * C::PB + nq) = v[p];
  }
};

// ------------------------------------------------------------- MFMA core
// Lane layout of v_mfma_f32_16x16x4_f32: lane l supplies A[l%16][l/16] and
// B[l/16][l%16]; D element (i, j) lives in lane j + 16*(i/4), register i%4.
// K-steps [kt0, kt1) of the product (kt1 < 0: to the end of K).
template <class C, class LA, class LB, class ST>
__device__ __forceinline__ void gemm_run(LA& la, LB& lb, const ST& store, int64_t M, int64_t N,
                                         int64_t K, int64_t m0, int64_t n0, int64_t kt0 = 0,
                                         int64_t kt1 = -1) {
  __shared__ __align__(16) float As[2][kBK * C::PA];
  __shared__ __align__(16) float Bs[2][kBK * C::PB];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave / C::WAVES_N) * C::WM, wn = (wave % C::WAVES_N) * C::WN;
  v4f acc[C::WTM][C::WTN];
#pragma unroll
  for (int i = 0; i < C::WTM; ++i)
#pragma unroll
    for (int j = 0; j < C::WTN; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  const int64_t nk = kt1 < 0 ? ceil_div(K, kBK) : kt1;
  la.fetch(kt0 * kBK);
  lb.fetch(kt0 * kBK);
  la.stash(As[0]);
  lb.stash(Bs[0]);
  __syncthreads();
  for (int64_t kt = kt0; kt < nk; ++kt) {
    const int buf = static_cast<int>((kt - kt0) & 1);
    const bool more = kt + 1 < nk;
    if (more) {
      la.fetch((kt + 1) * kBK);
      lb.fetch((kt + 1) * kBK);
    }
    const float* as = As[buf];
    const float* bs = Bs[buf];
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 4) {
      const int k = kk + (lane >> 4);
      float a[C::WTM], b[C::WTN];
#pragma unroll
      for (int i = 0; i < C::WTM; ++i) a[i] = as[k * C::PA + wm + i * 16 + (lane & 15)];
#pragma unroll
      for (int j = 0; j < C::WTN; ++j) b[j] = bs[k * C::PB + wn + j * 16 + (lane & 15)];
#pragma unroll
      for (int i = 0; i < C::WTM; ++i)
#pragma unroll
        for (int j = 0; j < C::WTN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      la.stash(As[buf ^ 1]);
      lb.stash(Bs[buf ^ 1]);
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < C::WTM; ++i)
#pragma unroll
    for (int j = 0; j < C::WTN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm + i * 16 + (lane >> 4) * 4 + r;
        const int64_t n = n0 + wn + j * 16 + (lane & 15);
        if (m < M && n < N) store(m, n, acc[i][j][r]);
      }
}

// ------------------------------------------------------------------ GEMM
struct GemmArgs {
  const void* a;
  int a_dt;
  int64_t a_si, a_sj;  // element strides of A [M, K]
  const void* b;
  int b_dt;
  int64_t b_si, b_sj;  // element strides of B [K, N]
  Dequant dq;          // B's dequantisation (per column or per tensor)
  float* out;
  int64_t som, son;
  BatchMap bm;
  int64_t M, N, K;
  float alpha;
  const int* only_if;  // the launch does nothing unless *only_if is set (NULL: always runs)
  // split-K: blockIdx.z = batch * splits + split; with splits > 1 each
  // split stores its raw partial tile at part[((b*splits + split)*M + m)*N + n]
  // and gemm_splitk_reduce forms out
  int splits;
  float* part;
  const void* bpack;   // B packed by kk_gemm_pack (the bf16 matrix-core path), or NULL
};

// A kinds: 0 = K-contiguous quads of TA, 1 = scalar gather.
// B kinds: 0 = N-contiguous quads of TB, 1 = scalar gather.
template <class C, int AK, int BK, typename TA, typename TB>
__global__ void __launch_bounds__(kNT) gemm_kernel(GemmArgs G) {
  if (G.only_if && *G.only_if == 0) return;
  const int splits = G.splits > 1 ? G.splits : 1;
  const int64_t bz = blockIdx.z / splits;
  const int split = static_cast<int>(blockIdx.z % splits);
  const int64_t oa = batch_offset(G.bm, 0, bz), ob = batch_offset(G.bm, 1, bz),
                oo = batch_offset(G.bm, 2, bz);
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * C::BM;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * C::BN;
  float* out = G.out + oo;
  const float alpha = G.alpha;
  const int64_t som = G.som, son = G.son;
  const int64_t M = G.M, N = G.N, K = G.K;
  float* part = splits > 1 ? G.part + ((bz * splits + split) * M) * N : nullptr;
  auto store = [&](int64_t m, int64_t n, float v) {
    if (part) part[m * N + n] = v;
    else out[m * som + n * son] = alpha == 1.0f ? v : v * alpha;
  };
  const Dequant none{};  // fp32 activations: no per-row dequantisation
  // this split's K-steps
  const int64_t nk_all = ceil_div(K, kBK), chunk = ceil_div(nk_all, splits);
  const int64_t kt0 = split * chunk, kt1 = std::min<int64_t>(nk_all, kt0 + chunk);
  auto getA = [&](int64_t m, int64_t k) -> float {
    if (m >= M || k >= K) return 0.0f;
    return load_as_f32(G.a, G.a_dt, oa + m * G.a_si + k * G.a_sj);
  };
  auto getB = [&](int64_t k, int64_t n) -> float {
    if (k >= K || n >= N) return 0.0f;
    const float q = load_as_f32(G.b, G.b_dt, ob + k * G.b_si + n * G.b_sj);
    return G.dq.active ? dequant_value(q, G.dq, n) : q;
  };
  if constexpr (AK == 0 && BK == 0) {
    AQuad<C, TA> la;
    la.init(static_cast<const TA*>(G.a) + oa, G.a_si, M, K, m0, none);
    BQuad<C, TB> lb;
    lb.init(static_cast<const TB*>(G.b) + ob, G.b_si, N, K, n0, G.dq);
    gemm_run<C>(la, lb, store, M, N, K, m0, n0, kt0, kt1);
  } else if constexpr (AK == 0) {
    AQuad<C, TA> la;
    la.init(static_cast<const TA*>(G.a) + oa, G.a_si, M, K, m0, none);
    if (G.b_si == 1) {
      BScalar<C, decltype(getB), false> lb{getB, n0};
      gemm_run<C>(la, lb, store, M, N, K, m0, n0, kt0, kt1);
    } else {
      BScalar<C, decltype(getB), true> lb{getB, n0};
      gemm_run<C>(la, lb, store, M, N, K, m0, n0, kt0, kt1);
    }
  } else if constexpr (BK == 0) {
    BQuad<C, TB> lb;
    lb.init(static_cast<const TB*>(G.b) + ob, G.b_si, N, K, n0, G.dq);
    if (G.a_si == 1) {
      AScalar<C, decltype(getA), false> la{getA, m0};
      gemm_run<C>(la, lb, store, M, N, K, m0, n0, kt0, kt1);
    } else {
      AScalar<C, decltype(getA), true> la{getA, m0};
      gemm_run<C>(la, lb, store, M, N, K, m0, n0, kt0, kt1);
    }
  } else {
    // consecutive threads walk the unit-stride direction of each operand
    if (G.a_si == 1) {
      AScalar<C, decltype(getA), false> la{getA, m0};
      if (G.b_si == 1) {
        BScalar<C, decltype(getB), false> lb{getB, n0};
        gemm_run<C>(la, lb, store, M, N, K, m0, n0, kt0, kt1);
      } else {
        BScalar<C, decltype(getB), true> lb{getB, n0};
        gemm_run<C>(la, lb, store, M, N, K, m0, n0, kt0, kt1);
      }
    } else {
      AScalar<C, decltype(getA), true> la{getA, m0};
      if (G.b_si == 1) {
        BScalar<C, decltype(getB), false> lb{getB, n0};
        gemm_run<C>(la, lb, store, M, N, K, m0, n0, kt0, kt1);
      } else {
        BScalar<C, decltype(getB), true> lb{getB, n0};
        gemm_run<C>(la, lb, store, M, N, K, m0, n0, kt0, kt1);
      }
    }
  }
}

// ------------------------------------------------------------------ conv
struct ConvArgs {
  const void* w;       // [Cout, Cin*Kw] (K contiguous)
  int w_dt;
  Dequant dq;          // per output channel (row) or per tensor
  const float* x;      // [N, Cin, L]
  float* out;          // [N, Cout, Lout]
  const float* bias;   // [Cout] or NULL
  int64_t Cin, L, Kw, s, d, p0, Lout;
  int64_t M, K;        // Cout, Cin*Kw
};

// AK: 0 = quad loads of TW (K % 4 == 0), 1 = scalar gather.
template <class C, int AK, typename TW>
__global__ void __launch_bounds__(kNT) conv1d_kernel(ConvArgs A) {
  const int64_t bz = blockIdx.z;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * C::BM;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * C::BN;
  const int64_t M = A.M, N = A.Lout, K = A.K;
  float* out = A.out + bz * M * N;
  const float* bias = A.bias;
  auto store = [&](int64_t m, int64_t n, float v) { out[m * N + n] = bias ? v + bias[m] : v; };
  BIm2col<C> lb;
  lb.x = A.x + bz * A.Cin * A.L;
  lb.L = A.L; lb.Kw = A.Kw; lb.s = A.s; lb.d = A.d; lb.p0 = A.p0; lb.Kdim = K; lb.Lout = N;
  lb.r0 = threadIdx.x / BIm2col<C>::QPR;
  lb.l0 = n0 + (threadIdx.x % BIm2col<C>::QPR) * 4;
  if constexpr (AK == 0) {
    AQuad<C, TW> la;
    la.init(static_cast<const TW*>(A.w), K, M, K, m0, A.dq);
    gemm_run<C>(la, lb, store, M, N, K, m0, n0);
  } else {
    auto getA = [&](int64_t m, int64_t k) -> float {
      if (m >= M || k >= K) return 0.0f;
      const float q = load_as_f32(A.w, A.w_dt, m * K + k);
      return A.dq.active ? dequant_value(q, A.dq, m) : q;
    };
    AScalar<C, decltype(getA), true> la{getA, m0};
    gemm_run<C>(la, lb, store, M, N, K, m0, n0);
  }
}

// out[b][m][n] = the splits' partials summed in split order, then alpha.
__global__ void __launch_bounds__(256) gemm_splitk_reduce(GemmArgs G, int64_t batch) {
  const int64_t MN = G.M * G.N, total = batch * MN;
  const int S = G.splits;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t bz = i / MN, mn = i - bz * MN;
    const int64_t m = mn / G.N, n = mn - m * G.N;
    const float* p = G.part + bz * S * MN + mn;
    float v = p[0];
    for (int s = 1; s < S; ++s) v = v + p[s * MN];
    const int64_t o = batch_offset(G.bm, 2, bz) + m * G.som + n * G.son;
    G.out[o] = G.alpha == 1.0f ? v : v * G.alpha;
  }
}

// ------------------------------------------------- transposed conv (phases)
// For output phase r (uncropped positions j = q*s + r):
//   out[co, q*s + r] = sum_{ci, m} W[ci, co, r + s*m] * x[ci, q - m]
// A[co, kk] = W[ci, co, r + s*m] and B[kk, q] = x[ci, q - m], kk = ci*MR + m.
struct ConvTArgs {
  const void* w;       // [Cin, Cout, Kw]
  int w_dt;
  Dequant dq;          // per output channel or per tensor
  const float* x;      // [N, Cin, L]
  float* out;          // [N, Cout, Lout]
  const float* bias;
  int64_t Cin, Cout, L, Kw, s, MR, p0, Lout, nq;
};

template <class C>
__global__ void __launch_bounds__(kNT) conv_transpose_kernel(ConvTArgs A) {
  const int64_t r = blockIdx.z % A.s;
  const int64_t bz = blockIdx.z / A.s;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * C::BM;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * C::BN;
  const int64_t M = A.Cout, N = A.nq, K = A.Cin * A.MR;
  const float* x = A.x + bz * A.Cin * A.L;
  float* out = A.out + bz * A.Cout * A.Lout;
  const int64_t s = A.s, p0 = A.p0, Lout = A.Lout, MR = A.MR, Kw = A.Kw, L = A.L;
  const float* bias = A.bias;
  auto store = [&](int64_t m, int64_t q, float v) {
    const int64_t jo = q * s + r - p0;
    if (jo >= 0 && jo < Lout) out[m * Lout + jo] = bias ? v + bias[m] : v;
  };
  auto getA = [&](int64_t co, int64_t kk) -> float {
    if (co >= M || kk >= K) return 0.0f;
    const int64_t ci = kk / MR, mt = kk - ci * MR;
    const int64_t k = r + s * mt;
    if (k >= Kw) return 0.0f;
    const float q = load_as_f32(A.w, A.w_dt, (ci * M + co) * Kw + k);
    return A.dq.active ? dequant_value(q, A.dq, co) : q;
  };
  auto getB = [&](int64_t kk, int64_t q) -> float {
    if (kk >= K || q >= N) return 0.0f;
    const int64_t ci = kk / MR, mt = kk - ci * MR;
    const int64_t l = q - mt;
    if (l < 0 || l >= L) return 0.0f;
    return x[ci * L + l];
  };
  AScalar<C, decltype(getA), false> la{getA, m0};
  BScalar<C, decltype(getB), true> lb{getB, n0};
  gemm_run<C>(la, lb, store, M, N, K, m0, n0);
}

// --------------------------------------------------- direct conv kernels
// Any group / dilation: one thread per output element, fp32 FMA.
struct DirectArgs {
  const float* x;
  const void* w;
  int w_dt;
  Dequant dq;
  const float* bias;
  float* out;
  int64_t N, Cin, L, Cout, K, Lout, s, d, p0, group;
};

__global__ void conv1d_direct_kernel(DirectArgs D) {
  const int64_t total = D.N * D.Cout * D.Lout;
  const int64_t cin_g = D.Cin / D.group, cout_g = D.Cout / D.group;
  for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t l = t % D.Lout;
    const int64_t co = (t / D.Lout) % D.Cout;
    const int64_t n = t / (D.Lout * D.Cout);
    const int64_t g = co / cout_g;
    float acc = 0.0f;
    for (int64_t ci = 0; ci < cin_g; ++ci) {
      const float* xr = D.x + (n * D.Cin + g * cin_g + ci) * D.L;
      for (int64_t k = 0; k < D.K; ++k) {
        const int64_t pos = l * D.s + k * D.d - D.p0;
        if (pos < 0 || pos >= D.L) continue;
        float w = load_as_f32(D.w, D.w_dt, (co * cin_g + ci) * D.K + k);
        if (D.dq.active) w = dequant_value(w, D.dq, co);
        acc = __builtin_fmaf(w, xr[pos], acc);
      }
    }
    D.out[t] = D.bias ? acc + D.bias[co] : acc;
  }
}

__global__ void conv_transpose_direct_kernel(DirectArgs D) {
  // Here Cin/Cout are those of the transposed conv, w is [Cin, Cout/g, K].
  const int64_t total = D.N * D.Cout * D.Lout;
  const int64_t cin_g = D.Cin / D.group, cout_g = D.Cout / D.group;
  for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t jo = t % D.Lout;
    const int64_t co = (t / D.Lout) % D.Cout;
    const int64_t n = t / (D.Lout * D.Cout);
    const int64_t g = co / cout_g, coi = co % cout_g;
    const int64_t j = jo + D.p0;
    const int64_t q0 = j / D.s, r0 = j - q0 * D.s;
    float acc = 0.0f;
    for (int64_t cl = 0; cl < cin_g; ++cl) {
      const int64_t ci = g * cin_g + cl;
      const float* xr = D.x + (n * D.Cin + ci) * D.L;
      if (D.d == 1) {  // the taps k = r0, r0 + s, ... (j = q0 s + r0) read x[q0], x[q0 - 1], ...
        for (int64_t k = r0, l = q0; k < D.K && l >= 0; k += D.s, --l) {
          if (l >= D.L) continue;
          float w = load_as_f32(D.w, D.w_dt, (ci * cout_g + coi) * D.K + k);
          if (D.dq.active) w = dequant_value(w, D.dq, co);
          acc = __builtin_fmaf(w, xr[l], acc);
        }
        continue;
      }
      for (int64_t k = 0; k < D.K; ++k) {
        const int64_t num = j - k * D.d;
        if (num < 0 || num % D.s) continue;
        const int64_t l = num / D.s;
        if (l >= D.L) continue;
        float w = load_as_f32(D.w, D.w_dt, (ci * cout_g + coi) * D.K + k);
        if (D.dq.active) w = dequant_value(w, D.dq, co);
        acc = __builtin_fmaf(w, xr[l], acc);
      }
    }
    D.out[t] = D.bias ? acc + D.bias[co] : acc;
  }
}

// Tall, skinny products (N <= 4 columns, K <= 32): a thread per row of A,
// its K values in registers, B's few values from cache.  The tiled kernel
// would spend a 32- or 64-wide tile on each column here ([2154000, 9] x
// [9, 1] in the harmonic source's Linear).
constexpr int kSkinnyK = 32, kSkinnyN = 4;

__global__ void __launch_bounds__(256) gemm_skinny_kernel(GemmArgs G, int64_t batch) {
  if (G.only_if && *G.only_if == 0) return;
  const int64_t rows = batch * G.M;
  const int K = static_cast<int>(G.K), N = static_cast<int>(G.N);
  for (int64_t r = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; r < rows;
       r += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t bz = r / G.M, m = r % G.M;
    const int64_t oa = batch_offset(G.bm, 0, bz), ob = batch_offset(G.bm, 1, bz),
                  oo = batch_offset(G.bm, 2, bz);
    float a[kSkinnyK];
#pragma unroll
    for (int k = 0; k < kSkinnyK; ++k) {
      a[k] = 0.0f;
      if (k < K) {
        a[k] = load_as_f32(G.a, G.a_dt, oa + m * G.a_si + k * G.a_sj);
      }
    }
#pragma unroll
    for (int n = 0; n < kSkinnyN; ++n) {
      if (n >= N) break;
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < kSkinnyK; ++k) {
        if (k >= K) break;
        float b = load_as_f32(G.b, G.b_dt, ob + k * G.b_si + n * G.b_sj);
        if (G.dq.active) b = dequant_value(b, G.dq, n);
        acc = __builtin_fmaf(a[k], b, acc);
      }
      G.out[oo + m * G.som + n * G.son] = G.alpha == 1.0f ? acc : acc * G.alpha;
    }
  }
}

// ConvTranspose1d with few output channels, group 1, dilation 1 (the
// iSTFT's 22 -> 1): the dequantised weights in LDS, a thread per output
// walking only its taps (k = j mod s, + s, ...), the same order of terms as
// the direct kernel above.
constexpr int kSmallTW = 4096;  // weights held in LDS

__global__ void __launch_bounds__(256) conv_transpose_small_kernel(DirectArgs D) {
  __shared__ float ws[kSmallTW];
  const int nw = static_cast<int>(D.Cin * D.Cout * D.K);
  for (int i = threadIdx.x; i < nw; i += blockDim.x) {
    float w = load_as_f32(D.w, D.w_dt, i);
    if (D.dq.active) w = dequant_value(w, D.dq, (i / static_cast<int>(D.K)) % static_cast<int>(D.Cout));
    ws[i] = w;
  }
  __syncthreads();
  const int K = static_cast<int>(D.K), s = static_cast<int>(D.s), Cout = static_cast<int>(D.Cout);
  const int64_t total = D.N * D.Cout * D.Lout;
  for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t jo = t % D.Lout;
    const int64_t nco = t / D.Lout;
    const int co = static_cast<int>(nco % D.Cout);
    const int64_t n = nco / D.Cout;
    const int64_t j = jo + D.p0;
    const int64_t q0 = j / s;
    const int r0 = static_cast<int>(j - q0 * s);
    const float* xn = D.x + n * D.Cin * D.L;
    float acc = 0.0f;
    for (int ci = 0; ci < static_cast<int>(D.Cin); ++ci) {
      const float* xr = xn + ci * D.L;
      const float* wr = ws + (ci * Cout + co) * K;
      int64_t l = q0;
      for (int k = r0; k < K && l >= 0; k += s, --l)
        if (l < D.L) acc = __builtin_fmaf(wr[k], xr[l], acc);
    }
    D.out[t] = D.bias ? acc + D.bias[co] : acc;
  }
}

// ------------------------------------------------------------- launching
enum TileSize { TILE_L = 0, TILE_M = 1, TILE_S = 2 };

// The largest tile that still gives every SIMD (4 per CU) a wavefront; the
// smallest tile otherwise.
static TileSize pick_tile(int64_t M, int64_t N, int64_t batch) {
  const int64_t simds = 4 * static_cast<int64_t>(ctx().num_cus > 0 ? ctx().num_cus : 256);
  const int64_t wl = ceil_div(M, 64) * ceil_div(N, 64) * batch * 4;
  if (wl >= simds) return TILE_L;
  const int64_t wm = ceil_div(M, 64) * ceil_div(N, 32) * batch * 4;
  if (wm >= simds) return TILE_M;
  return TILE_S;
}

static dim3 grid_of(TileSize t, int64_t M, int64_t N, int64_t z) {
  const int bm = t == TILE_S ? 32 : 64, bn = t == TILE_L ? 64 : 32;
  return dim3(static_cast<unsigned>(ceil_div(N, bn)), static_cast<unsigned>(ceil_div(M, bm)),
              static_cast<unsigned>(z));
}

static int check_grid(const dim3& g, int64_t z) {
  if (z > 65535 || g.y > 65535)
    return set_error(KK_E_UNSUPPORTED, "grid %u x %u x %lld too large", g.x, g.y, (long long)z);
  return KK_OK;
}

#define KK_TILED(KERNEL, TS, GRID, ...)                                                       \
  do {                                                                                          \
    if ((TS) == TILE_L)                                                                         \
      KK_LAUNCH((KERNEL<CfgL, __VA_ARGS__>), GRID, dim3(kNT), 0, ctx().stream, args); \
    else if ((TS) == TILE_M)                                                                    \
      KK_LAUNCH((KERNEL<CfgM, __VA_ARGS__>), GRID, dim3(kNT), 0, ctx().stream, args); \
    else                                                                                        \
      KK_LAUNCH((KERNEL<CfgS, __VA_ARGS__>), GRID, dim3(kNT), 0, ctx().stream, args); \
  } while (0)

static bool aligned(const void* p, int bytes) {
  return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

static int conv_common(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                       const kk_tensor* bias, const char* who) {
  KK_TRY(require_ready());
  KK_TRY(check_tensor(out, "out"));
  KK_TRY(check_tensor(x, "x"));
  KK_TRY(check_tensor(w, "w"));
  if (x->rank != 3 || w->rank != 3 || out->rank != 3)
    return set_error(KK_E_ARG, "%s: x, w and out must be rank 3", who);
  if (x->dtype != KK_F32 || out->dtype != KK_F32)
    return set_error(KK_E_ARG, "%s: x and out must be fp32", who);
  if (!is_contiguous(x) || !is_contiguous(out) || !is_contiguous(w))
    return set_error(KK_E_ARG, "%s: x, w and out must be contiguous", who);
  if (bias) {
    KK_TRY(check_tensor(bias, "bias"));
    if (bias->dtype != KK_F32 || !is_contiguous(bias))
      return set_error(KK_E_ARG, "%s: bias must be contiguous fp32", who);
  }
  return KK_OK;
}

// weights_rounded: keep numpy's per-weight rounding of (q - zp) * scale
// (the fp32 matrix cores); else 8-bit and fp16 weights may take the bf16
// matrix cores, which scale the exact sum instead.
static int launch_gemm(const GemmArgs& args, int64_t batch, bool weights_rounded = false) {
  if (args.N <= kSkinnyN && args.K <= kSkinnyK && args.M * batch >= 4096) {
    const int64_t rows = args.M * batch;
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>(ceil_div(rows, 256), 1 << 16));
    KK_LAUNCH(gemm_skinny_kernel, dim3(grid), dim3(256), 0, ctx().stream, args, batch);
    return check_launch("gemm_skinny_kernel");
  }
  // 8-bit and fp16 weights with fp32 activations: the bf16 matrix cores
  // with split activations (fp32 accuracy)
  if (!weights_rounded && args.a_dt == KK_F32 && args.a_sj == 1 && args.b_sj == 1) {
    int st = KK_OK;
    if (gemm_dq_try(static_cast<const float*>(args.a), args.a_si, args.b, args.b_dt, args.b_si,
                    args.dq, args.out, args.som, args.son, args.bm, args.M, args.N, args.K, batch,
                    args.alpha, args.only_if, args.bpack, &st))
      return st;
  }
  const TileSize ts = pick_tile(args.M, args.N, batch);
  dim3 grid = grid_of(ts, args.M, args.N, batch);
  KK_TRY(check_grid(grid, batch));
  // Split K when the tiles leave CUs idle and the K loop is long (each
  // K-step waits on its loads): partials in the context scratch, summed in
  // split order by a second kernel.
  GemmArgs args_s = args;
  {
    const int64_t cus = ctx().num_cus > 0 ? ctx().num_cus : 256;
    const int64_t blocks = static_cast<int64_t>(grid.x) * grid.y * grid.z;
    const int64_t nk = ceil_div(args.K, kBK);
    int64_t S = 1;
    while (S < 8 && blocks * S < 2 * cus && nk / (2 * S) >= 4 &&
           static_cast<size_t>(batch * 2 * S * args.M * args.N) * 4 <= kScratchBytes &&
           batch * 2 * S <= 65535)
      S *= 2;
    if (S > 1) {
      args_s.splits = static_cast<int>(S);
      args_s.part = static_cast<float*>(ctx().scratch);
      grid.z = static_cast<unsigned>(batch * S);
    }
  }
  const GemmArgs& args0 = args;
  {
  const GemmArgs& args = args_s;
  // Vector paths: A fp32 with K contiguous; B with N contiguous; rows (and
  // batch strides) whole 4-element groups, aligned to them.
  const int bsz = dtype_size(args.b_dt);
  bool a_quad = args.a_dt == KK_F32 && args.a_sj == 1 && args.K % 4 == 0 &&
                args.a_si % 4 == 0 && aligned(args.a, 16);
  bool b_quad = args.b_sj == 1 && args.N % 4 == 0 && args.b_si % 4 == 0 && aligned(args.b, 4 * bsz);
  for (int d = 0; d < args.bm.nb; ++d) {
    if (args.bm.st[0][d] % 4) a_quad = false;
    if (args.bm.st[1][d] % 4) b_quad = false;
  }
  if (a_quad && b_quad) {
    switch (args.b_dt) {
      case KK_F32: KK_TILED(gemm_kernel, ts, grid, 0, 0, float, float); break;
      case KK_F16: KK_TILED(gemm_kernel, ts, grid, 0, 0, float, __half); break;
      case KK_I8: KK_TILED(gemm_kernel, ts, grid, 0, 0, float, int8_t); break;
      default: KK_TILED(gemm_kernel, ts, grid, 0, 0, float, uint8_t); break;
    }
  } else if (a_quad) {
    KK_TILED(gemm_kernel, ts, grid, 0, 1, float, float);
  } else if (b_quad) {
    switch (args.b_dt) {
      case KK_F32: KK_TILED(gemm_kernel, ts, grid, 1, 0, float, float); break;
      case KK_F16: KK_TILED(gemm_kernel, ts, grid, 1, 0, float, __half); break;
      case KK_I8: KK_TILED(gemm_kernel, ts, grid, 1, 0, float, int8_t); break;
      default: KK_TILED(gemm_kernel, ts, grid, 1, 0, float, uint8_t); break;
    }
  } else {
    KK_TILED(gemm_kernel, ts, grid, 1, 1, float, float);
  }
  KK_TRY(check_launch("gemm_kernel"));
  if (args.splits > 1) {
    const int64_t total = batch * args.M * args.N;
    KK_LAUNCH(gemm_splitk_reduce, dim3(static_cast<unsigned>(std::min<int64_t>(ceil_div(total, 256), 4096))),
                       dim3(256), 0, ctx().stream, args, batch);
    KK_TRY(check_launch("gemm_splitk_reduce"));
  }
  }
  (void)args0;
  return KK_OK;
}


int matmul_shape(const kk_tensor* out, const kk_tensor* a, const kk_tensor* w, BatchMap* bm,
                 int64_t* M_, int64_t* N_, int64_t* K_, int64_t* batch_out, const char* who) {
  KK_TRY(require_ready());
  KK_TRY(check_tensor(out, "out"));
  KK_TRY(check_tensor(a, "a"));
  KK_TRY(check_tensor(w, "w"));
  if (a->rank < 2 || w->rank < 2 || out->rank < 2)
    return set_error(KK_E_ARG, "%s: operands need rank >= 2 (promote vectors first)", who);
  const int64_t M = a->shape[a->rank - 2], K = a->shape[a->rank - 1];
  const int64_t K2 = w->shape[w->rank - 2], N = w->shape[w->rank - 1];
  if (K != K2)
    return set_error(KK_E_ARG, "%s: inner extents differ (%lld vs %lld)", who, (long long)K,
                     (long long)K2);
  if (out->shape[out->rank - 2] != M || out->shape[out->rank - 1] != N)
    return set_error(KK_E_ARG, "%s: out must end in [%lld, %lld]", who, (long long)M,
                     (long long)N);
  const int nb = out->rank - 2;
  if (nb > 6) return set_error(KK_E_UNSUPPORTED, "%s: more than 6 batch axes", who);
  if (a->rank - 2 > nb || w->rank - 2 > nb)
    return set_error(KK_E_ARG, "%s: operand has more batch axes than out", who);
  int64_t batch = 1;
  bm->nb = nb;
  for (int i = 0; i < nb; ++i) {
    const int64_t od = out->shape[i];
    bm->dims[i] = od;
    bm->st[2][i] = out->strides[i];
    batch *= od;
    const kk_tensor* ops[2] = {a, w};
    for (int k = 0; k < 2; ++k) {
      const int pad = nb - (ops[k]->rank - 2);
      if (i < pad) { bm->st[k][i] = 0; continue; }
      const int64_t d = ops[k]->shape[i - pad];
      if (d == od) bm->st[k][i] = ops[k]->strides[i - pad];
      else if (d == 1) bm->st[k][i] = 0;
      else return set_error(KK_E_ARG, "%s: batch axis %d does not broadcast", who, i);
    }
  }
  *M_ = M; *N_ = N; *K_ = K;
  *batch_out = batch;
  return KK_OK;
}

// Shapes, batch broadcasting and strides of out = a @ w (numpy matmul rules
// for rank >= 2 operands).  Leaves the dequantisation to the caller.
static int setup_gemm(GemmArgs* G, const kk_tensor* out, const kk_tensor* a, const kk_tensor* w,
                      int64_t* batch_out, const char* who) {
  KK_TRY(matmul_shape(out, a, w, &G->bm, &G->M, &G->N, &G->K, batch_out, who));
  G->a = a->data; G->a_dt = a->dtype;
  G->a_si = a->strides[a->rank - 2]; G->a_sj = a->strides[a->rank - 1];
  G->b = w->data; G->b_dt = w->dtype;
  G->b_si = w->strides[w->rank - 2]; G->b_sj = w->strides[w->rank - 1];
  G->out = static_cast<float*>(out->data);
  G->som = out->strides[out->rank - 2];
  G->son = out->strides[out->rank - 1];
  G->alpha = 1.0f;
  return KK_OK;
}

int zp_shift(Dequant* d, const kk_tensor* zp, int64_t count, const char* who) {
  *d = Dequant();
  if (!zp) return KK_OK;
  KK_TRY(check_tensor(zp, "zero point"));
  if (!(zp->dtype == KK_I8 || zp->dtype == KK_U8 || zp->dtype == KK_I32))
    return set_error(KK_E_ARG, "%s: zero point must be int8/uint8/int32", who);
  const int64_t n = numel(zp);
  if (n != 1 && n != count)
    return set_error(KK_E_ARG, "%s: zero point has %lld elements, expected 1 or %lld", who,
                     (long long)n, (long long)count);
  if (n > 1 && !is_contiguous(zp))
    return set_error(KK_E_ARG, "%s: per-column zero point must be contiguous", who);
  d->zp = zp->data;
  d->zp_dt = zp->dtype;
  d->zp_stride = n > 1 ? 1 : 0;
  d->active = true;
  return KK_OK;
}

// fp16 / 8-bit-weight convolutions on the fp16 matrix cores (kk_conv_f16.hip):
// true when that path ran (its status in *rc), false when it does not apply.
bool convh_run(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w, const Dequant& dq,
               const kk_tensor* bias, bool transposed, int64_t stride, int64_t dilation,
               int64_t pad0, int64_t Nq, const kk_tensor* packed, int* rc);
int convh_check_packed(const kk_tensor* packed, const kk_tensor* w, const kk_tensor* w_zp,
                       bool transposed, int64_t stride, const char* who);

int gemm(const kk_tensor* out, const kk_tensor* a, const kk_tensor* w, const kk_tensor* w_scale,
         const kk_tensor* w_zp, float alpha, bool weights_rounded, const kk_tensor* packed) {
  const char* who = packed ? "kk_gemm_packed" : "kk_gemm";
  GemmArgs G{};
  int64_t batch = 0;
  KK_TRY(setup_gemm(&G, out, a, w, &batch, who));
  if (!is_float(a->dtype)) return set_error(KK_E_ARG, "%s: a must be f32/f16", who);
  if (out->dtype != KK_F32) return set_error(KK_E_ARG, "%s: out must be fp32", who);
  KK_TRY(make_dequant(&G.dq, w, w_scale, w_zp, G.N, who));
  if (packed) {
    KK_TRY(gemm_check_packed(packed, w, w_zp, who));
    G.bpack = packed->data;
  }
  G.alpha = alpha;
  if (G.M == 0 || G.N == 0 || batch == 0) return KK_OK;
  if (G.K == 0) return kk_fill(out, 0.0);
  return launch_gemm(G, batch, weights_rounded);
}

}  // namespace kk

using namespace kk;

extern "C" {

int kk_gemm(const kk_tensor* out, const kk_tensor* a, const kk_tensor* w, const kk_tensor* w_scale,
            const kk_tensor* w_zp, float alpha) {
  return gemm(out, a, w, w_scale, w_zp, alpha, false, nullptr);
}

int kk_gemm_packed(const kk_tensor* out, const kk_tensor* a, const kk_tensor* w,
                   const kk_tensor* packed, const kk_tensor* w_scale, const kk_tensor* w_zp,
                   float alpha) {
  KK_TRY(check_tensor(w, "w"));
  return gemm(out, a, w, w_scale, w_zp, alpha, false, packed);
}

}  // extern "C"

namespace kk {

// Conv1d (ref_runtime.py:58-82, 101-103); `packed` (checked by the caller)
// holds w laid out by kk_conv_pack, or NULL.
static int conv1d_impl(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                       const kk_tensor* w_scale, const kk_tensor* w_zp, const kk_tensor* bias,
                       int stride, int dilation, int pad0, int pad1, int group,
                       const kk_tensor* packed, const char* who) {
  KK_TRY(conv_common(out, x, w, bias, who));
  const int64_t N = x->shape[0], Cin = x->shape[1], L = x->shape[2];
  const int64_t Cout = w->shape[0], cin_g = w->shape[1], K = w->shape[2];
  if (stride < 1 || dilation < 1 || pad0 < 0 || pad1 < 0 || group < 1)
    return set_error(KK_E_ARG, "%s: bad stride/dilation/pads/group", who);
  if (Cin % group || Cout % group || cin_g * group != Cin)
    return set_error(KK_E_ARG, "%s: channels do not match group %d", who, group);
  const int64_t span = static_cast<int64_t>(dilation) * (K - 1) + 1;
  const int64_t Lp = L + pad0 + pad1;
  const int64_t Lout = Lp >= span ? (Lp - span) / stride + 1 : 0;
  if (out->shape[0] != N || out->shape[1] != Cout || out->shape[2] != Lout)
    return set_error(KK_E_ARG, "%s: out must be [%lld, %lld, %lld]", who, (long long)N,
                     (long long)Cout, (long long)Lout);
  if (bias && numel(bias) != Cout) return set_error(KK_E_ARG, "%s: bias needs Cout elements", who);
  Dequant dq;
  KK_TRY(make_dequant(&dq, w, w_scale, w_zp, Cout, who));
  if (packed) {
    if (group != 1) return set_error(KK_E_ARG, "%s: packed weights need group 1", who);
    KK_TRY(convh_check_packed(packed, w, w_zp, false, stride, who));
  }
  if (N * Cout * Lout == 0) return KK_OK;
  const float* bp = bias ? static_cast<const float*>(bias->data) : nullptr;
  if (group == 1) {
    // fp16 / 8-bit weights: the fp16 matrix cores when they apply
    int rc = KK_OK;
    if (convh_run(out, x, w, dq, bias, false, stride, dilation, pad0, Lout, packed, &rc)) return rc;
    ConvArgs args{};
    args.w = w->data; args.w_dt = w->dtype; args.dq = dq;
    args.x = static_cast<const float*>(x->data);
    args.out = static_cast<float*>(out->data);
    args.bias = bp;
    args.Cin = Cin; args.L = L; args.Kw = K; args.s = stride; args.d = dilation; args.p0 = pad0;
    args.Lout = Lout; args.M = Cout; args.K = Cin * K;
    const TileSize ts = pick_tile(Cout, Lout, N);
    const dim3 grid = grid_of(ts, Cout, Lout, N);
    KK_TRY(check_grid(grid, N));
    const bool quad = (Cin * K) % 4 == 0 && aligned(w->data, 4 * dtype_size(w->dtype));
    if (!quad) {
      KK_TILED(conv1d_kernel, ts, grid, 1, float);
    } else {
      switch (w->dtype) {
        case KK_F32: KK_TILED(conv1d_kernel, ts, grid, 0, float); break;
        case KK_F16: KK_TILED(conv1d_kernel, ts, grid, 0, __half); break;
        case KK_I8: KK_TILED(conv1d_kernel, ts, grid, 0, int8_t); break;
        default: KK_TILED(conv1d_kernel, ts, grid, 0, uint8_t); break;
      }
    }
    return check_launch("conv1d_kernel");
  }
  DirectArgs D{};
  D.x = static_cast<const float*>(x->data); D.w = w->data; D.w_dt = w->dtype; D.dq = dq;
  D.bias = bp; D.out = static_cast<float*>(out->data);
  D.N = N; D.Cin = Cin; D.L = L; D.Cout = Cout; D.K = K; D.Lout = Lout;
  D.s = stride; D.d = dilation; D.p0 = pad0; D.group = group;
  const int64_t total = N * Cout * Lout;
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>(ceil_div(total, 256), 1 << 20));
  KK_LAUNCH(conv1d_direct_kernel, dim3(grid), dim3(256), 0, ctx().stream, D);
  return check_launch("conv1d_direct_kernel");
}

// ConvTranspose1d (ref_runtime.py:83-99); `packed` as for conv1d_impl.
static int conv_transpose1d_impl(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                                 const kk_tensor* w_scale, const kk_tensor* w_zp,
                                 const kk_tensor* bias, int stride, int dilation, int pad0,
                                 int pad1, int group, int output_padding,
                                 const kk_tensor* packed, const char* who) {
  KK_TRY(conv_common(out, x, w, bias, who));
  const int64_t N = x->shape[0], Cin = x->shape[1], L = x->shape[2];
  const int64_t cout_g = w->shape[1], K = w->shape[2];
  if (stride < 1 || dilation < 1 || pad0 < 0 || pad1 < 0 || group < 1 || output_padding < 0)
    return set_error(KK_E_ARG, "%s: bad stride/dilation/pads/group", who);
  if (w->shape[0] != Cin || Cin % group)
    return set_error(KK_E_ARG, "%s: w must be [Cin, Cout/group, K]", who);
  const int64_t Cout = cout_g * group;
  const int64_t lfull = (L - 1) * stride + static_cast<int64_t>(dilation) * (K - 1) + 1 + output_padding;
  const int64_t Lout = lfull - pad0 - pad1;
  if (L < 1 || Lout < 0) return set_error(KK_E_ARG, "%s: empty or negative output", who);
  if (out->shape[0] != N || out->shape[1] != Cout || out->shape[2] != Lout)
    return set_error(KK_E_ARG, "%s: out must be [%lld, %lld, %lld]", who, (long long)N,
                     (long long)Cout, (long long)Lout);
  if (bias && numel(bias) != Cout)
    return set_error(KK_E_ARG, "%s: bias needs Cout elements", who);
  Dequant dq;
  KK_TRY(make_dequant(&dq, w, w_scale, w_zp, Cout, who));
  if (packed) {
    if (group != 1 || dilation != 1)
      return set_error(KK_E_ARG, "%s: packed weights need group 1 and dilation 1", who);
    KK_TRY(convh_check_packed(packed, w, w_zp, true, stride, who));
  }
  if (N * Cout * Lout == 0) return KK_OK;
  const float* bp = bias ? static_cast<const float*>(bias->data) : nullptr;
  // A few output channels: the direct kernel (a thread per output, only the
  // taps that land on it); the tiles below would be mostly empty rows.
  if (group == 1 && dilation == 1 && (Cout > 4 || packed)) {
    // Phase decomposition: s sub-GEMMs of MR = ceil(K/s) taps each.  Output
    // position jo maps to j = jo + p0 = q*s + r; every q up to the last
    // needed j is enumerated (x reads are bounds-checked, so the
    // output_padding tail gets the bias alone).
    const int64_t jmax = lfull - pad1 - 1;  // last needed uncropped position
    const int64_t nq = jmax / stride + 1;
    // fp16 / 8-bit weights: the fp16 matrix cores when they apply
    int rc = KK_OK;
    if (convh_run(out, x, w, dq, bias, true, stride, 1, pad0, nq, packed, &rc)) return rc;
    ConvTArgs args{};
    args.w = w->data; args.w_dt = w->dtype; args.dq = dq;
    args.x = static_cast<const float*>(x->data);
    args.out = static_cast<float*>(out->data); args.bias = bp;
    args.Cin = Cin; args.Cout = Cout; args.L = L; args.Kw = K; args.s = stride;
    args.MR = ceil_div(K, stride); args.p0 = pad0; args.Lout = Lout;
    args.nq = nq;
    const TileSize ts = pick_tile(Cout, args.nq, N * stride);
    const dim3 grid = grid_of(ts, Cout, args.nq, N * stride);
    KK_TRY(check_grid(grid, N * stride));
    if (ts == TILE_L)
      KK_LAUNCH(conv_transpose_kernel<CfgL>, grid, dim3(kNT), 0, ctx().stream, args);
    else if (ts == TILE_M)
      KK_LAUNCH(conv_transpose_kernel<CfgM>, grid, dim3(kNT), 0, ctx().stream, args);
    else
      KK_LAUNCH(conv_transpose_kernel<CfgS>, grid, dim3(kNT), 0, ctx().stream, args);
    return check_launch("conv_transpose_kernel");
  }
  DirectArgs D{};
  D.x = static_cast<const float*>(x->data); D.w = w->data; D.w_dt = w->dtype; D.dq = dq;
  D.bias = bp; D.out = static_cast<float*>(out->data);
  D.N = N; D.Cin = Cin; D.L = L; D.Cout = Cout; D.K = K; D.Lout = Lout;
  D.s = stride; D.d = dilation; D.p0 = pad0; D.group = group;
  const int64_t total = N * Cout * Lout;
  if (group == 1 && dilation == 1 && Cin * Cout * K <= kSmallTW) {
    const unsigned g = static_cast<unsigned>(std::min<int64_t>(ceil_div(total, 256), 2048));
    KK_LAUNCH(conv_transpose_small_kernel, dim3(g), dim3(256), 0, ctx().stream, D);
    return check_launch("conv_transpose_small_kernel");
  }
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>(ceil_div(total, 256), 1 << 20));
  KK_LAUNCH(conv_transpose_direct_kernel, dim3(grid), dim3(256), 0, ctx().stream, D);
  return check_launch("conv_transpose_direct_kernel");
}

}  // namespace kk

extern "C" {

int kk_conv1d(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w, const kk_tensor* w_scale,
              const kk_tensor* w_zp, const kk_tensor* bias, int stride, int dilation, int pad0,
              int pad1, int group) {
  return conv1d_impl(out, x, w, w_scale, w_zp, bias, stride, dilation, pad0, pad1, group, nullptr,
                     "kk_conv1d");
}

int kk_conv1d_packed(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                     const kk_tensor* packed, const kk_tensor* w_scale, const kk_tensor* w_zp,
                     const kk_tensor* bias, int stride, int dilation, int pad0, int pad1) {
  if (!packed) return set_error(KK_E_ARG, "kk_conv1d_packed: packed is required");
  return conv1d_impl(out, x, w, w_scale, w_zp, bias, stride, dilation, pad0, pad1, 1, packed,
                     "kk_conv1d_packed");
}

int kk_conv_transpose1d(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                        const kk_tensor* w_scale, const kk_tensor* w_zp, const kk_tensor* bias,
                        int stride, int dilation, int pad0, int pad1, int group,
                        int output_padding) {
  return conv_transpose1d_impl(out, x, w, w_scale, w_zp, bias, stride, dilation, pad0, pad1, group,
                               output_padding, nullptr, "kk_conv_transpose1d");
}

int kk_conv_transpose1d_packed(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                               const kk_tensor* packed, const kk_tensor* w_scale,
                               const kk_tensor* w_zp, const kk_tensor* bias, int stride, int pad0,
                               int pad1, int output_padding) {
  if (!packed) return set_error(KK_E_ARG, "kk_conv_transpose1d_packed: packed is required");
  return conv_transpose1d_impl(out, x, w, w_scale, w_zp, bias, stride, 1, pad0, pad1, 1,
                               output_padding, packed, "kk_conv_transpose1d_packed");
}

}  // extern "C"
