// Contractions: batched MatMul with weight dequantisation, Conv1d as an
// implicit GEMM and ConvTranspose1d as a phase-decomposed implicit GEMM, all
// on one fp32 MFMA core (v_mfma_f32_16x16x4_f32: fp32 operands, exact fp32
// products, fp32 accumulation -- the fp32 semantics of the numpy reference).
//
// Core: a block computes a BM x BN tile of C = A . B with BK = 16 deep
// K-steps.  Each wavefront owns a 32 x 32 sub-tile made of 2 x 2 MFMA
// 16 x 16 tiles.  A and B tiles are fetched from global memory by loader
// policies (dense strided, int8/uint8 dequant, im2col gather, transposed-conv
// phase gather) into registers, dequantised to fp32 there, stored K-major in
// LDS, and the next tile's fetch overlaps the current tile's MFMAs.
#include <algorithm>

#include "kk_internal.h"

namespace kk {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kBK = 16;
constexpr int kPad = 4;  // LDS row padding (floats) against bank conflicts

// Batch offsets: up to 6 batch axes with per-operand strides (0 = broadcast).
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

// ----------------------------------------------------------- loader: dense
// Element (i, j) of a strided matrix, i over `rows`, j over `cols`, with
// optional dequantisation by column (`deq_by_col`) or by row.
struct DenseLoader {
  const void* p;
  int dt;
  int64_t si, sj;      // element strides
  int64_t rows, cols;  // logical extents (for bounds)
  Dequant dq;
  int deq_by_col;      // 1: scale/zp index = j, 0: = i
  int which;           // batch stride slot
  __device__ __forceinline__ float get(int64_t boff, int64_t i, int64_t j) const {
    if (i >= rows || j >= cols) return 0.0f;
    const int64_t off = boff + i * si + j * sj;
    float v;
    if (dt == KK_F32) v = static_cast<const float*>(p)[off];
    else v = load_as_f32(p, dt, off);
    if (dq.active) v = dequant_value(v, dq, deq_by_col ? j : i);
    return v;
  }
};

// --------------------------------------------------------- loader: im2col
// B[kk, l] = x[n, ci, l*s + k*d - p0] with kk = ci*K + k (zero padding).
struct Im2colLoader {
  const float* x;
  int64_t cin, L, K, s, d, p0;
  int64_t rows, cols;  // Cin*K, Lout
  __device__ __forceinline__ float get(int64_t boff, int64_t kk, int64_t l) const {
    if (kk >= rows || l >= cols) return 0.0f;
    const int64_t ci = kk / K, k = kk - ci * K;
    const int64_t pos = l * s + k * d - p0;
    if (pos < 0 || pos >= L) return 0.0f;
    return x[boff + ci * L + pos];
  }
};

// ------------------------------------------- loaders: transposed-conv phase
// For output phase r (positions j = q*s + r of the uncropped output):
//   out[co, q*s + r] = sum_{ci, m} W[ci, co, r + s*m] * x[ci, q - m]
// A[co, kk] = W[ci, co, r + s*m] and B[kk, q] = x[ci, q - m], kk = ci*MR + m.
struct ConvTWLoader {
  const void* w;
  int dt;
  Dequant dq;
  int64_t cout_g, K, s, MR;
  int64_t rows, cols;  // Cout, Cin*MR
  __device__ __forceinline__ float get(int64_t r, int64_t co, int64_t kk) const {
    if (co >= rows || kk >= cols) return 0.0f;
    const int64_t ci = kk / MR, m = kk - ci * MR;
    const int64_t k = r + s * m;
    if (k >= K) return 0.0f;
    float v = load_as_f32(w, dt, (ci * cout_g + co) * K + k);
    if (dq.active) v = dequant_value(v, dq, co);
    return v;
  }
};
struct ConvTXLoader {
  const float* x;
  int64_t L, MR;
  int64_t rows, cols;  // Cin*MR, number of q
  int64_t q0;          // first q of this phase
  __device__ __forceinline__ float get(int64_t boff, int64_t kk, int64_t qi) const {
    if (kk >= rows || qi >= cols) return 0.0f;
    const int64_t ci = kk / MR, m = kk - ci * MR;
    const int64_t l = q0 + qi - m;
    if (l < 0 || l >= L) return 0.0f;
    return x[boff + ci * L + l];
  }
};

// ------------------------------------------------------------ MFMA core
// acc[2][2] are the wave's four 16x16 tiles.  Lane layout of
// v_mfma_f32_16x16x4_f32: lane l supplies A[l%16][l/16] and B[l/16][l%16];
// D element (i, j) lives in lane j + 16*(i/4), register i%4.
template <int BM, int BN>
struct Tile {
  static constexpr int WN = BN / 32;
  static constexpr int WAVES = (BM / 32) * (BN / 32);
  static constexpr int NT = WAVES * 64;
  static constexpr int AE = BM * kBK / NT;  // A elements per thread
  static constexpr int BE = kBK * BN / NT;  // B elements per thread
};

template <int BM, int BN>
__device__ __forceinline__ void mfma_tile(const float* As, const float* Bs, v4f (&acc)[2][2],
                                          int wm, int wn, int lane) {
#pragma unroll
  for (int kk = 0; kk < kBK; kk += 4) {
    const int k = kk + (lane >> 4);
    float a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) a[i] = As[k * (BM + kPad) + wm + i * 16 + (lane & 15)];
#pragma unroll
    for (int j = 0; j < 2; ++j) b[j] = Bs[k * (BN + kPad) + wn + j * 16 + (lane & 15)];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
  }
}

// Element e of a tile with `fast` extent along the contiguous direction.
// A tile is BM (m) x kBK (k); B tile is kBK (k) x BN (n).  `a_kfast`: A's
// consecutive elements run along k (else along m); `b_nfast` likewise.

// Generic kernel body.  GetA(boffA/phase, m, k) and GetB(boffB, k, n) return
// fp32 values; Store(m, n, value) writes the result.
template <int BM, int BN, class FA, class FB, class FS>
__device__ __forceinline__ void gemm_body(const FA& getA, const FB& getB, const FS& store,
                                          int64_t M, int64_t N, int64_t K, bool a_kfast,
                                          bool b_nfast) {
  using T = Tile<BM, BN>;
  __shared__ float As[2][kBK * (BM + kPad)];
  __shared__ float Bs[2][kBK * (BN + kPad)];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = (wave / T::WN) * 32, wn = (wave % T::WN) * 32;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * BM;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * BN;

  v4f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  float ra[T::AE], rb[T::BE];
  auto fetch = [&](int64_t k0) {
#pragma unroll
    for (int t = 0; t < T::AE; ++t) {
      const int e = tid + t * T::NT;
      const int mi = a_kfast ? e / kBK : e % BM;
      const int ki = a_kfast ? e % kBK : e / BM;
      ra[t] = (k0 + ki < K) ? getA(m0 + mi, k0 + ki) : 0.0f;
    }
#pragma unroll
    for (int t = 0; t < T::BE; ++t) {
      const int e = tid + t * T::NT;
      const int ni = b_nfast ? e % BN : e / kBK;
      const int ki = b_nfast ? e / BN : e % kBK;
      rb[t] = (k0 + ki < K) ? getB(k0 + ki, n0 + ni) : 0.0f;
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int t = 0; t < T::AE; ++t) {
      const int e = tid + t * T::NT;
      const int mi = a_kfast ? e / kBK : e % BM;
      const int ki = a_kfast ? e % kBK : e / BM;
      As[buf][ki * (BM + kPad) + mi] = ra[t];
    }
#pragma unroll
    for (int t = 0; t < T::BE; ++t) {
      const int e = tid + t * T::NT;
      const int ni = b_nfast ? e % BN : e / kBK;
      const int ki = b_nfast ? e / BN : e % kBK;
      Bs[buf][ki * (BN + kPad) + ni] = rb[t];
    }
  };

  const int64_t nk = ceil_div(K, kBK);
  fetch(0);
  stash(0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int buf = static_cast<int>(kt & 1);
    if (kt + 1 < nk) fetch((kt + 1) * kBK);
    mfma_tile<BM, BN>(As[buf], Bs[buf], acc, wm, wn, lane);
    if (kt + 1 < nk) stash(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm + i * 16 + (lane >> 4) * 4 + r;
        const int64_t n = n0 + wn + j * 16 + (lane & 15);
        if (m < M && n < N) store(m, n, acc[i][j][r]);
      }
}

// ------------------------------------------------------------------ GEMM
struct GemmArgs {
  DenseLoader a, b;
  float* out;
  int64_t som, son;
  BatchMap bm;
  int64_t M, N, K;
  float alpha;
  int a_kfast, b_nfast;
};

template <int BM, int BN>
__global__ void __launch_bounds__((BM / 32) * (BN / 32) * 64) gemm_kernel(GemmArgs G) {
  const int64_t b = blockIdx.z;
  const int64_t oa = batch_offset(G.bm, 0, b), ob = batch_offset(G.bm, 1, b),
                oo = batch_offset(G.bm, 2, b);
  auto getA = [&](int64_t m, int64_t k) { return G.a.get(oa, m, k); };
  auto getB = [&](int64_t k, int64_t n) { return G.b.get(ob, k, n); };
  float* out = G.out + oo;
  const float alpha = G.alpha;
  auto store = [&](int64_t m, int64_t n, float v) {
    out[m * G.som + n * G.son] = alpha == 1.0f ? v : v * alpha;
  };
  gemm_body<BM, BN>(getA, getB, store, G.M, G.N, G.K, G.a_kfast, G.b_nfast);
}

// ------------------------------------------------------------------ conv
struct ConvArgs {
  DenseLoader w;       // A = W as [Cout, Cin*K], dequant by row (co)
  Im2colLoader x;      // B
  float* out;          // [N, Cout, Lout]
  const float* bias;   // [Cout] or NULL
  int64_t x_bstride;   // Cin*L
  int64_t o_bstride;   // Cout*Lout
  int64_t M, N, K;
};

template <int BM, int BN>
__global__ void __launch_bounds__((BM / 32) * (BN / 32) * 64) conv1d_kernel(ConvArgs C) {
  const int64_t b = blockIdx.z;
  const int64_t ox = b * C.x_bstride;
  auto getA = [&](int64_t m, int64_t k) { return C.w.get(0, m, k); };
  auto getB = [&](int64_t k, int64_t n) { return C.x.get(ox, k, n); };
  float* out = C.out + b * C.o_bstride;
  const int64_t N = C.N;
  const float* bias = C.bias;
  auto store = [&](int64_t m, int64_t n, float v) {
    out[m * N + n] = bias ? v + bias[m] : v;
  };
  gemm_body<BM, BN>(getA, getB, store, C.M, C.N, C.K, true, true);
}

struct ConvTArgs {
  ConvTWLoader w;
  ConvTXLoader x;
  float* out;          // [N, Cout, Lout]
  const float* bias;
  int64_t x_bstride, o_bstride;
  int64_t s, p0, Lout, lfull;
  int64_t M, K;        // Cout, Cin*MR
  int64_t nq;          // q values per phase (upper bound)
};

template <int BM, int BN>
__global__ void __launch_bounds__((BM / 32) * (BN / 32) * 64) conv_transpose_kernel(ConvTArgs C) {
  const int64_t r = blockIdx.z % C.s;
  const int64_t b = blockIdx.z / C.s;
  const int64_t ox = b * C.x_bstride;
  ConvTXLoader xl = C.x;
  auto getA = [&](int64_t m, int64_t k) { return C.w.get(r, m, k); };
  auto getB = [&](int64_t k, int64_t n) { return xl.get(ox, k, n); };
  float* out = C.out + b * C.o_bstride;
  const int64_t s = C.s, p0 = C.p0, Lout = C.Lout;
  const float* bias = C.bias;
  auto store = [&](int64_t m, int64_t q, float v) {
    const int64_t jo = q * s + r - p0;
    if (jo >= 0 && jo < Lout) out[m * Lout + jo] = bias ? v + bias[m] : v;
  };
  gemm_body<BM, BN>(getA, getB, store, C.M, C.nq, C.K, false, true);
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
    float acc = 0.0f;
    for (int64_t cl = 0; cl < cin_g; ++cl) {
      const int64_t ci = g * cin_g + cl;
      const float* xr = D.x + (n * D.Cin + ci) * D.L;
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

// ------------------------------------------------------------- launching
static int tiles_for(int64_t M, int64_t N, int64_t batch, int* bm, int* bn) {
  // Prefer 64x64 tiles; drop to smaller tiles while the grid would leave
  // most of the 256 CUs idle.
  const int64_t cus = ctx().num_cus > 0 ? ctx().num_cus : 256;
  const int64_t b64 = ceil_div(M, 64) * ceil_div(N, 64) * batch;
  if (b64 >= 2 * cus) { *bm = 64; *bn = 64; return KK_OK; }
  const int64_t b3264 = ceil_div(M, 32) * ceil_div(N, 64) * batch;
  if (b3264 >= 2 * cus) { *bm = 32; *bn = 64; return KK_OK; }
  *bm = 32; *bn = 32;
  return KK_OK;
}

#define KK_LAUNCH_TILED(KERNEL, BM, BN, GRID, ARGS)                                            \
  do {                                                                                          \
    if ((BM) == 64 && (BN) == 64)                                                               \
      hipLaunchKernelGGL((KERNEL<64, 64>), GRID, dim3(Tile<64, 64>::NT), 0, ctx().stream, ARGS); \
    else if ((BM) == 32 && (BN) == 64)                                                          \
      hipLaunchKernelGGL((KERNEL<32, 64>), GRID, dim3(Tile<32, 64>::NT), 0, ctx().stream, ARGS); \
    else                                                                                        \
      hipLaunchKernelGGL((KERNEL<32, 32>), GRID, dim3(Tile<32, 32>::NT), 0, ctx().stream, ARGS); \
  } while (0)

static int check_grid(int64_t gx, int64_t gy, int64_t gz) {
  if (gx > 0x7fffffff || gy > 65535 || gz > 65535)
    return set_error(KK_E_UNSUPPORTED, "grid %lld x %lld x %lld too large", (long long)gx,
                     (long long)gy, (long long)gz);
  return KK_OK;
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

}  // namespace kk

using namespace kk;

extern "C" {

int kk_gemm(const kk_tensor* out, const kk_tensor* a, const kk_tensor* w, const kk_tensor* w_scale,
            const kk_tensor* w_zp, float alpha) {
  KK_TRY(require_ready());
  KK_TRY(check_tensor(out, "out"));
  KK_TRY(check_tensor(a, "a"));
  KK_TRY(check_tensor(w, "w"));
  if (a->rank < 2 || w->rank < 2 || out->rank < 2)
    return set_error(KK_E_ARG, "kk_gemm: operands need rank >= 2 (promote vectors first)");
  if (!is_float(a->dtype)) return set_error(KK_E_ARG, "kk_gemm: a must be f32/f16");
  if (out->dtype != KK_F32) return set_error(KK_E_ARG, "kk_gemm: out must be fp32");
  const int64_t M = a->shape[a->rank - 2], K = a->shape[a->rank - 1];
  const int64_t K2 = w->shape[w->rank - 2], N = w->shape[w->rank - 1];
  if (K != K2) return set_error(KK_E_ARG, "kk_gemm: inner extents differ (%lld vs %lld)",
                                (long long)K, (long long)K2);
  if (out->shape[out->rank - 2] != M || out->shape[out->rank - 1] != N)
    return set_error(KK_E_ARG, "kk_gemm: out must end in [%lld, %lld]", (long long)M, (long long)N);
  GemmArgs G{};
  KK_TRY(make_dequant(&G.b.dq, w, w_scale, w_zp, N, "kk_gemm"));
  // Batch axes: numpy broadcasting of a[:-2] and w[:-2] against out[:-2].
  const int nb = out->rank - 2;
  if (nb > 6) return set_error(KK_E_UNSUPPORTED, "kk_gemm: more than 6 batch axes");
  if (a->rank - 2 > nb || w->rank - 2 > nb)
    return set_error(KK_E_ARG, "kk_gemm: operand has more batch axes than out");
  int64_t batch = 1;
  G.bm.nb = nb;
  for (int i = 0; i < nb; ++i) {
    const int64_t od = out->shape[i];
    G.bm.dims[i] = od;
    G.bm.st[2][i] = out->strides[i];
    batch *= od;
    const kk_tensor* ops[2] = {a, w};
    for (int k = 0; k < 2; ++k) {
      const int pad = nb - (ops[k]->rank - 2);
      if (i < pad) { G.bm.st[k][i] = 0; continue; }
      const int64_t d = ops[k]->shape[i - pad];
      if (d == od) G.bm.st[k][i] = ops[k]->strides[i - pad];
      else if (d == 1) G.bm.st[k][i] = 0;
      else return set_error(KK_E_ARG, "kk_gemm: batch axis %d does not broadcast", i);
    }
  }
  if (M == 0 || N == 0 || batch == 0) return KK_OK;
  G.a.p = a->data; G.a.dt = a->dtype;
  G.a.si = a->strides[a->rank - 2]; G.a.sj = a->strides[a->rank - 1];
  G.a.rows = M; G.a.cols = K;
  G.b.p = w->data; G.b.dt = w->dtype;
  G.b.si = w->strides[w->rank - 2]; G.b.sj = w->strides[w->rank - 1];
  G.b.rows = K; G.b.cols = N; G.b.deq_by_col = 1;
  G.out = static_cast<float*>(out->data);
  G.som = out->strides[out->rank - 2];
  G.son = out->strides[out->rank - 1];
  G.M = M; G.N = N; G.K = K;
  G.alpha = alpha;
  // Coalesce each fetch along the operand's unit-stride direction.
  G.a_kfast = (G.a.sj == 1) || (G.a.si != 1);
  G.b_nfast = (G.b.sj == 1) || (G.b.si != 1);
  if (K == 0) return kk_fill(out, 0.0);
  int bm, bn;
  tiles_for(M, N, batch, &bm, &bn);
  const int64_t gx = ceil_div(N, bn), gy = ceil_div(M, bm);
  KK_TRY(check_grid(gx, gy, batch));
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy), static_cast<unsigned>(batch));
  KK_LAUNCH_TILED(gemm_kernel, bm, bn, grid, G);
  return check_launch("gemm_kernel");
}

int kk_conv1d(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w, const kk_tensor* w_scale,
              const kk_tensor* w_zp, const kk_tensor* bias, int stride, int dilation, int pad0,
              int pad1, int group) {
  KK_TRY(conv_common(out, x, w, bias, "kk_conv1d"));
  const int64_t N = x->shape[0], Cin = x->shape[1], L = x->shape[2];
  const int64_t Cout = w->shape[0], cin_g = w->shape[1], K = w->shape[2];
  if (stride < 1 || dilation < 1 || pad0 < 0 || pad1 < 0 || group < 1)
    return set_error(KK_E_ARG, "kk_conv1d: bad stride/dilation/pads/group");
  if (Cin % group || Cout % group || cin_g * group != Cin)
    return set_error(KK_E_ARG, "kk_conv1d: channels do not match group %d", group);
  const int64_t span = static_cast<int64_t>(dilation) * (K - 1) + 1;
  const int64_t Lp = L + pad0 + pad1;
  const int64_t Lout = Lp >= span ? (Lp - span) / stride + 1 : 0;
  if (out->shape[0] != N || out->shape[1] != Cout || out->shape[2] != Lout)
    return set_error(KK_E_ARG, "kk_conv1d: out must be [%lld, %lld, %lld]", (long long)N,
                     (long long)Cout, (long long)Lout);
  if (bias && numel(bias) != Cout) return set_error(KK_E_ARG, "kk_conv1d: bias needs Cout elements");
  Dequant dq;
  KK_TRY(make_dequant(&dq, w, w_scale, w_zp, Cout, "kk_conv1d"));
  if (N * Cout * Lout == 0) return KK_OK;
  const float* bp = bias ? static_cast<const float*>(bias->data) : nullptr;
  if (group == 1) {
    ConvArgs C{};
    C.w.p = w->data; C.w.dt = w->dtype; C.w.si = cin_g * K; C.w.sj = 1;
    C.w.rows = Cout; C.w.cols = Cin * K; C.w.dq = dq; C.w.deq_by_col = 0;
    C.x.x = static_cast<const float*>(x->data);
    C.x.cin = Cin; C.x.L = L; C.x.K = K; C.x.s = stride; C.x.d = dilation; C.x.p0 = pad0;
    C.x.rows = Cin * K; C.x.cols = Lout;
    C.out = static_cast<float*>(out->data);
    C.bias = bp;
    C.x_bstride = Cin * L;
    C.o_bstride = Cout * Lout;
    C.M = Cout; C.N = Lout; C.K = Cin * K;
    int bm, bn;
    tiles_for(Cout, Lout, N, &bm, &bn);
    const int64_t gx = ceil_div(Lout, bn), gy = ceil_div(Cout, bm);
    KK_TRY(check_grid(gx, gy, N));
    const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy), static_cast<unsigned>(N));
    KK_LAUNCH_TILED(conv1d_kernel, bm, bn, grid, C);
    return check_launch("conv1d_kernel");
  }
  DirectArgs D{};
  D.x = static_cast<const float*>(x->data); D.w = w->data; D.w_dt = w->dtype; D.dq = dq;
  D.bias = bp; D.out = static_cast<float*>(out->data);
  D.N = N; D.Cin = Cin; D.L = L; D.Cout = Cout; D.K = K; D.Lout = Lout;
  D.s = stride; D.d = dilation; D.p0 = pad0; D.group = group;
  const int64_t total = N * Cout * Lout;
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>(ceil_div(total, 256), 1 << 20));
  hipLaunchKernelGGL(conv1d_direct_kernel, dim3(grid), dim3(256), 0, ctx().stream, D);
  return check_launch("conv1d_direct_kernel");
}

int kk_conv_transpose1d(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                        const kk_tensor* w_scale, const kk_tensor* w_zp, const kk_tensor* bias,
                        int stride, int dilation, int pad0, int pad1, int group,
                        int output_padding) {
  KK_TRY(conv_common(out, x, w, bias, "kk_conv_transpose1d"));
  const int64_t N = x->shape[0], Cin = x->shape[1], L = x->shape[2];
  const int64_t cout_g = w->shape[1], K = w->shape[2];
  if (stride < 1 || dilation < 1 || pad0 < 0 || pad1 < 0 || group < 1 || output_padding < 0)
    return set_error(KK_E_ARG, "kk_conv_transpose1d: bad stride/dilation/pads/group");
  if (w->shape[0] != Cin || Cin % group)
    return set_error(KK_E_ARG, "kk_conv_transpose1d: w must be [Cin, Cout/group, K]");
  const int64_t Cout = cout_g * group;
  const int64_t lfull = (L - 1) * stride + static_cast<int64_t>(dilation) * (K - 1) + 1 + output_padding;
  const int64_t Lout = lfull - pad0 - pad1;
  if (L < 1 || Lout < 0) return set_error(KK_E_ARG, "kk_conv_transpose1d: empty or negative output");
  if (out->shape[0] != N || out->shape[1] != Cout || out->shape[2] != Lout)
    return set_error(KK_E_ARG, "kk_conv_transpose1d: out must be [%lld, %lld, %lld]", (long long)N,
                     (long long)Cout, (long long)Lout);
  if (bias && numel(bias) != Cout)
    return set_error(KK_E_ARG, "kk_conv_transpose1d: bias needs Cout elements");
  Dequant dq;
  KK_TRY(make_dequant(&dq, w, w_scale, w_zp, Cout, "kk_conv_transpose1d"));
  if (N * Cout * Lout == 0) return KK_OK;
  const float* bp = bias ? static_cast<const float*>(bias->data) : nullptr;
  if (group == 1 && dilation == 1) {
    // Phase decomposition: s sub-GEMMs of MR = ceil(K/s) taps each.  Output
    // position jo maps to j = jo + p0 = q*s + r.  Positions j >= (L-1)s+K
    // (output_padding tail) receive nothing but the bias, handled because
    // every q up to the last j is enumerated and x reads are bounds-checked.
    const int64_t MR = ceil_div(K, stride);
    ConvTArgs C{};
    C.w.w = w->data; C.w.dt = w->dtype; C.w.dq = dq; C.w.cout_g = cout_g; C.w.K = K;
    C.w.s = stride; C.w.MR = MR; C.w.rows = Cout; C.w.cols = Cin * MR;
    C.x.x = static_cast<const float*>(x->data); C.x.L = L; C.x.MR = MR; C.x.rows = Cin * MR;
    const int64_t jmax = lfull - pad1 - 1;  // last needed uncropped position
    C.nq = jmax / stride + 1;
    C.x.cols = C.nq; C.x.q0 = 0;
    C.out = static_cast<float*>(out->data); C.bias = bp;
    C.x_bstride = Cin * L; C.o_bstride = Cout * Lout;
    C.s = stride; C.p0 = pad0; C.Lout = Lout; C.lfull = lfull;
    C.M = Cout; C.K = Cin * MR;
    int bm, bn;
    tiles_for(Cout, C.nq, N * stride, &bm, &bn);
    const int64_t gx = ceil_div(C.nq, bn), gy = ceil_div(Cout, bm);
    KK_TRY(check_grid(gx, gy, N * stride));
    const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy),
                    static_cast<unsigned>(N * stride));
    KK_LAUNCH_TILED(conv_transpose_kernel, bm, bn, grid, C);
    return check_launch("conv_transpose_kernel");
  }
  DirectArgs D{};
  D.x = static_cast<const float*>(x->data); D.w = w->data; D.w_dt = w->dtype; D.dq = dq;
  D.bias = bp; D.out = static_cast<float*>(out->data);
  D.N = N; D.Cin = Cin; D.L = L; D.Cout = Cout; D.K = K; D.Lout = Lout;
  D.s = stride; D.d = dilation; D.p0 = pad0; D.group = group;
  const int64_t total = N * Cout * Lout;
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>(ceil_div(total, 256), 1 << 20));
  hipLaunchKernelGGL(conv_transpose_direct_kernel, dim3(grid), dim3(256), 0, ctx().stream, D);
  return check_launch("conv_transpose_direct_kernel");
}

}  // extern "C"
