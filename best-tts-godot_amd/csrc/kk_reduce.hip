// Row reductions and normalisations: ReduceMean/Sum/Max, InstanceNorm with
// the AdaIN affine (optionally with the style Linear fused in), LayerNorm /
// SkipLayerNorm and Softmax.
//
// Row kernels hold their row in registers: a GROUP of 64 (one wavefront) or
// 256 (four wavefronts) threads owns one row, each thread NV vectors of VEC
// floats, so the row is read from HBM once and written once.  Reductions
// are wave butterflies (__shfl_xor) plus, for 256-thread groups, a 4-entry
// LDS combine; the order is fixed, so results are identical run to run.
// Statistics follow numpy: mean = sum / n in fp32, variance two-pass
// mean((x - mean)^2), normalisation a true division by sqrt(var + eps).
#include <algorithm>
#include <numeric>
#include <utility>
#include <vector>

#include "kk_internal.h"

namespace kk {

constexpr int kRowBlock = 256;

// DPP: wave sums through DPP lane moves (kernels held to a tolerance); else
// the butterfly, whose order the numpy-order kernels rely on.
template <int GROUP, bool DPP = false>
__device__ __forceinline__ float group_sum(float v, float* lds) {
  v = DPP ? wave_sum_dpp(v) : wave_sum(v);
  if constexpr (GROUP == 64) {
    return v;
  } else {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) lds[w] = v;
    __syncthreads();
    return (lds[0] + lds[1]) + (lds[2] + lds[3]);
  }
}

template <int GROUP, bool DPP = false>
__device__ __forceinline__ float group_max(float v, float* lds) {
  v = DPP ? wave_max_dpp(v) : wave_max(v);
  if constexpr (GROUP == 64) {
    return v;
  } else {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) lds[w] = v;
    __syncthreads();
    return fmaxf(fmaxf(lds[0], lds[1]), fmaxf(lds[2], lds[3]));
  }
}

// Two independent group sums in one LDS round (each sum in group_sum's
// order, so the results are the same bits); lds holds 8 floats.
template <int GROUP, bool DPP = false>
__device__ __forceinline__ void group_sum_pair(float& a, float& b, float* lds) {
  a = DPP ? wave_sum_dpp(a) : wave_sum(a);
  b = DPP ? wave_sum_dpp(b) : wave_sum(b);
  if constexpr (GROUP != 64) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) {
      lds[w] = a;
      lds[4 + w] = b;
    }
    __syncthreads();
    a = (lds[0] + lds[1]) + (lds[2] + lds[3]);
    b = (lds[4] + lds[5]) + (lds[6] + lds[7]);
  }
}

// Loads this thread's share of a row of `n` floats into r[NV][VEC].
// Element index of (j, e) is (j * GROUP + g) * VEC + e; missing ones are 0.
// STREAM rows are read once (non-temporal); parameter vectors shared by
// every row (scale, bias) use ordinary cached loads.
template <int GROUP, int NV, int VEC, bool STREAM = true>
__device__ __forceinline__ void load_row(const float* __restrict__ row, int64_t n, int g,
                                         float (&r)[NV][VEC]) {
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t base = (static_cast<int64_t>(j) * GROUP + g) * VEC;
    if constexpr (VEC == 4) {
      if (base < n) {
        const float4 v = STREAM ? ld_stream4(row + base)
                                : *reinterpret_cast<const float4*>(row + base);
        r[j][0] = v.x; r[j][1] = v.y; r[j][2] = v.z; r[j][3] = v.w;
      } else {
        r[j][0] = r[j][1] = r[j][2] = r[j][3] = 0.0f;
      }
    } else {
      r[j][0] = base < n ? (STREAM ? ld_stream(row + base) : row[base]) : 0.0f;
    }
  }
}

template <int GROUP, int NV, int VEC>
__device__ __forceinline__ void store_row(float* __restrict__ row, int64_t n, int g,
                                          const float (&r)[NV][VEC]) {
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t base = (static_cast<int64_t>(j) * GROUP + g) * VEC;
    if (base < n) {
      if constexpr (VEC == 4) {
        st_stream4(row + base, make_float4(r[j][0], r[j][1], r[j][2], r[j][3]));
      } else {
        st_stream(row + base, r[j][0]);
      }
    }
  }
}

// Two-pass mean and variance of the row held in r (n valid elements; the
// padding lanes hold 0 and are masked out of the second pass).
template <int GROUP, int NV, int VEC, bool DPP = false>
__device__ __forceinline__ void row_stats(float (&r)[NV][VEC], int64_t n, int g, float* lds,
                                          float& mean, float& var) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int e = 0; e < VEC; ++e) s += r[j][e];
  s = group_sum<GROUP, DPP>(s, lds);
  mean = s / static_cast<float>(n);
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t base = (static_cast<int64_t>(j) * GROUP + g) * VEC;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float d = r[j][e] - mean;
      r[j][e] = d;  // keep x - mean for the output pass
      if (base + e < n) q += d * d;
    }
  }
  q = group_sum<GROUP, DPP>(q, lds);
  var = q / static_cast<float>(n);
}

// ----------------------------------------------------- InstanceNorm / AdaIN
// Style projection for channel c of C: h[j] = sum_k style[k] * W[k, j] + b[j]
// for j = c (gamma) and j = C + c (beta).  W is any-strided, optionally
// int8/uint8 with per-tensor/per-column dequantisation.
struct StyleArgs {
  const float* style;     // [S] fp32 (contiguous)
  const void* w;          // [S, 2C]
  int w_dt;
  int64_t w_sk, w_sj;     // strides of W in elements
  Dequant dq;
  const float* bias;      // [2C] or NULL
  int64_t S;
};

// This thread's share (k = g, g + GROUP, ...) of the two dot products.
template <int GROUP>
__device__ __forceinline__ void style_dots(const StyleArgs& sa, int64_t C, int64_t c, int g,
                                           float& ag, float& ab) {
  ag = 0.0f;
  ab = 0.0f;
  const int64_t jg = c, jb = C + c;
  for (int64_t k = g; k < sa.S; k += GROUP) {
    const float s = sa.style[k];
    float wg = load_as_f32(sa.w, sa.w_dt, k * sa.w_sk + jg * sa.w_sj);
    float wb = load_as_f32(sa.w, sa.w_dt, k * sa.w_sk + jb * sa.w_sj);
    if (sa.dq.active) {
      wg = dequant_value(wg, sa.dq, jg);
      wb = dequant_value(wb, sa.dq, jb);
    }
    ag = __builtin_fmaf(s, wg, ag);
    ab = __builtin_fmaf(s, wb, ab);
  }
}

template <int GROUP>
__device__ __forceinline__ void style_affine(const StyleArgs& sa, int64_t C, int64_t c, int g,
                                             float* lds, float& gamma, float& beta) {
  // the bias loads go out with the dot products' loads, not after the
  // block-wide sums (whose barriers keep the compiler from moving them up)
  float bg = 0.0f, bb = 0.0f;
  if (sa.bias) {
    bg = sa.bias[c];
    bb = sa.bias[C + c];
  }
  float ag, ab;
  style_dots<GROUP>(sa, C, c, g, ag, ab);
  group_sum_pair<GROUP, true>(ag, ab, lds);
  if (sa.bias) {
    ag = ag + bg;
    ab = ab + bb;
  }
  gamma = ag;
  beta = ab;
}

// Per-channel affine applied after the normalisation, and an optional
// LeakyRelu:
//   mode 0: y = q
//   mode 1: y = q * (gamma[c] + 1) + beta[c], gb = [gamma | beta] (2C)
//   mode 2: the same with (gamma, beta) = style . W + b computed in-kernel
//   mode 3: y = q * scale[c] + shift[c] (either may be NULL: 1 / 0), the
//           Mul/Add tail of the graph's InstanceNorm chain
// then, if leaky, y = y < 0 ? y * alpha : y (ref_runtime.py:476-479).
struct Affine {
  int mode;
  const float* gb;
  const float* scale;
  const float* shift;
  int leaky;
  float alpha;
  // optional snake after the affine: y + r * sin(a * y)^2, a and r per channel
  const float* snake_a;
  const float* snake_r;
};

struct RowAffine {
  float mul, add, sa, sr;
  bool has_mul, has_add;
};

__device__ __forceinline__ RowAffine row_affine(const Affine& af, int64_t C, int64_t c, float gamma,
                                                float beta) {
  RowAffine ra{1.0f, 0.0f, 0.0f, 0.0f, false, false};
  if (af.mode == 1 || af.mode == 2) {
    ra.mul = gamma + 1.0f; ra.add = beta; ra.has_mul = ra.has_add = true;
  } else if (af.mode == 3) {
    if (af.scale) { ra.mul = af.scale[c]; ra.has_mul = true; }
    if (af.shift) { ra.add = af.shift[c]; ra.has_add = true; }
  }
  if (af.snake_a) { ra.sa = af.snake_a[c]; ra.sr = af.snake_r[c]; }
  return ra;
}

// SNAKE false leaves the snake out of the code: kernels that hold whole
// rows in registers (the style-projected AdaIN) never take it, and sinf's
// slow path would make them spill.
template <bool SNAKE = true>
__device__ __forceinline__ float apply_affine(float q, const RowAffine& ra, const Affine& af) {
  float y = ra.has_mul ? q * ra.mul : q;
  if (ra.has_add) y = y + ra.add;
  if (af.leaky) y = y < 0.0f ? y * af.alpha : y;
  if (SNAKE && af.snake_a) {  // Mul(alpha, y) -> Sin -> Pow(., 2) -> Mul(recip, .) -> Add(y, .)
    y = y + ra.sr * kk_sin_sq(ra.sa * y);
  }
  return y;
}

template <int GROUP, int NV, int VEC>
__global__ void __launch_bounds__(kRowBlock) instnorm_kernel(float* __restrict__ out,
                                                             const float* __restrict__ x,
                                                             int64_t rows, int64_t C, int64_t T,
                                                             float eps, Affine af,
                                                             StyleArgs sa) {
  __shared__ float lds[8];
  const int RPB = blockDim.x / GROUP;  // 256 / GROUP, or 1 in 64-thread blocks
  const int g = threadIdx.x % GROUP;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / GROUP;
  // Every thread of the block takes part in the group reductions even when
  // its row is past the end (RPB > 1 only for GROUP == 64, whose reductions
  // are per wave, so the idle rows simply return).
  if constexpr (GROUP == 64) {
    if (row >= rows) return;
  }
  const int64_t c = row % C;
  // Issue the row's loads first so the style projection's latency hides
  // under them.
  const float* xr = x + row * T;
  float r[NV][VEC];
  load_row<GROUP, NV, VEC>(xr, T, g, r);
  float gamma = 0.0f, beta = 0.0f;
  if (af.mode == 2) style_affine<GROUP>(sa, C, c, g, lds, gamma, beta);
  else if (af.mode == 1) { gamma = af.gb[c]; beta = af.gb[C + c]; }
  const RowAffine ra = row_affine(af, C, c, gamma, beta);
  float mean, var;
  row_stats<GROUP, NV, VEC, true>(r, T, g, lds, mean, var);
  const float den = sqrtf(var + eps);
  if (af.mode == 2) {  // AdaIN (held to rel 1e-4): one division per row
    const float inv = 1.0f / den;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int e = 0; e < VEC; ++e) r[j][e] = apply_affine<false>(r[j][e] * inv, ra, af);
  } else {  // the InstanceNorm chain's own Div, per element
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int e = 0; e < VEC; ++e) r[j][e] = apply_affine<false>(r[j][e] / den, ra, af);
  }
  store_row<GROUP, NV, VEC>(out + row * T, T, g, r);
}

// AdaIN over one row per wave, for rows of 64 (NV - 1) < T / 4 <= 64 NV
// float4s (the decoder's [1,512,1200]): the row in registers, vectors
// 0 .. NV-2 whole for every lane (only the last one guarded), the three sums
// (style projection, mean, variance) DPP moves within the wave, the
// statistics scaled by 1 / T and normalised with the hardware reciprocal
// square root (within 1 ulp: AdaIN is held to rel 1e-4), and the output
// y = d * (inv * (gamma + 1)) + beta one FMA per element.  The
// generic row kernel's affine modes, LeakyRelu and per-element division
// cost it 841 VALU instructions a wave against ~160 here; with one wave on
// half the SIMDs, none of that overlapped anything.
template <int NV>
__global__ void __launch_bounds__(64) adain_row_kernel(float* __restrict__ out,
                                                      const float* __restrict__ x, int64_t C,
                                                      int T, float inv_t, float eps,
                                                      StyleArgs sa) {
  const int g = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t c = row % C;
  const float* __restrict__ xr = x + row * T;
  const bool tail = (NV - 1) * 64 + g < (T >> 2);  // this lane's last vector in the row
  float4 v[NV];
#pragma unroll
  for (int j = 0; j < NV - 1; ++j) v[j] = ld_stream4(xr + 4 * (j * 64 + g));
  v[NV - 1] = tail ? ld_stream4(xr + 4 * ((NV - 1) * 64 + g)) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  float bg = 0.0f, bb = 0.0f;
  if (sa.bias) {
    bg = sa.bias[c];
    bb = sa.bias[C + c];
  }
  float ag, ab;
  style_dots<64>(sa, C, c, g, ag, ab);
  const float mul = (wave_sum_dpp(ag) + bg) + 1.0f, add = wave_sum_dpp(ab) + bb;
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  const float mean = wave_sum_dpp(s) * inv_t;
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    v[j].x -= mean;
    v[j].y -= mean;
    v[j].z -= mean;
    v[j].w -= mean;
    float t = __builtin_fmaf(v[j].x, v[j].x, v[j].y * v[j].y);
    t = __builtin_fmaf(v[j].z, v[j].z, t);
    t = __builtin_fmaf(v[j].w, v[j].w, t);
    if (j < NV - 1 || tail) q += t;
  }
  const float inv = __builtin_amdgcn_rsqf(__builtin_fmaf(wave_sum_dpp(q), inv_t, eps));
  const float sc = inv * mul;
  float* __restrict__ orow = out + row * T;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const float4 y = make_float4(__builtin_fmaf(v[j].x, sc, add), __builtin_fmaf(v[j].y, sc, add),
                                 __builtin_fmaf(v[j].z, sc, add), __builtin_fmaf(v[j].w, sc, add));
    if (j < NV - 1 || tail) st_stream4(orow + 4 * (j * 64 + g), y);
  }
}

// AdaIN with NW waves per row (one row per block of 64 * NW threads), for
// rows long enough that 256 threads would each hold many vectors: more
// waves in flight per row and fewer registers per thread (at [1,512,9600],
// 8 waves per row run at 92% of a plain copy's rate against 83% for 4).
template <int NW>
__device__ __forceinline__ float wide_sum(float v, float* lds) {
  v = wave_sum_dpp(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) lds[w] = v;
  __syncthreads();
  float t[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) t[i] = lds[i];
#pragma unroll
  for (int h = NW / 2; h > 0; h /= 2)
#pragma unroll
    for (int i = 0; i < h; ++i) t[i] = t[i] + t[i + h];
  return t[0];
}

template <int NW>
__device__ __forceinline__ void wide_sum_pair(float& a, float& b, float* lds) {
  a = wave_sum_dpp(a);
  b = wave_sum_dpp(b);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) {
    lds[w] = a;
    lds[NW + w] = b;
  }
  __syncthreads();
  float t[NW], u[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    t[i] = lds[i];
    u[i] = lds[NW + i];
  }
#pragma unroll
  for (int h = NW / 2; h > 0; h /= 2)
#pragma unroll
    for (int i = 0; i < h; ++i) {
      t[i] = t[i] + t[i + h];
      u[i] = u[i] + u[i + h];
    }
  a = t[0];
  b = u[0];
}

template <int NW, int NV>
__global__ void __launch_bounds__(64 * NW) instnorm_wide_kernel(float* __restrict__ out,
                                                                const float* __restrict__ x,
                                                                int64_t C, int64_t T, float inv_t,
                                                                float eps, StyleArgs sa) {
  constexpr int G = 64 * NW;
  __shared__ float lds[2 * NW];
  const int g = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t c = row % C;
  float r[NV][4];
  load_row<G, NV, 4>(x + row * T, T, g, r);
  float bg = 0.0f, bb = 0.0f;  // issued before the barriers of the sums
  if (sa.bias) {
    bg = sa.bias[c];
    bb = sa.bias[C + c];
  }
  float ag, ab;
  style_dots<G>(sa, C, c, g, ag, ab);
  wide_sum_pair<NW>(ag, ab, lds);
  if (sa.bias) {
    ag = ag + bg;
    ab = ab + bb;
  }
  Affine af{};
  af.mode = 2;
  const RowAffine ra = row_affine(af, C, c, ag, ab);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) s += r[j][e];
  const float mean = wide_sum<NW>(s, lds) * inv_t;
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t base = (static_cast<int64_t>(j) * G + g) * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float d = r[j][e] - mean;
      r[j][e] = d;
      if (base + e < T) q += d * d;
    }
  }
  // the statistics scaled by 1 / T and the hardware reciprocal square root
  // (within 1 ulp: AdaIN is held to rel 1e-4)
  const float inv = __builtin_amdgcn_rsqf(__builtin_fmaf(wide_sum<NW>(q, lds), inv_t, eps));
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) r[j][e] = apply_affine<false>(r[j][e] * inv, ra, af);
  store_row<G, NV, 4>(out + row * T, T, g, r);
}

// Rows too long for registers: three passes over global memory.
__global__ void __launch_bounds__(kRowBlock) instnorm_long_kernel(float* __restrict__ out,
                                                                  const float* __restrict__ x,
                                                                  int64_t C, int64_t T, float eps,
                                                                  Affine af, StyleArgs sa) {
  __shared__ float lds[8];
  const int g = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t c = row % C;
  float gamma = 0.0f, beta = 0.0f;
  if (af.mode == 2) style_affine<kRowBlock>(sa, C, c, g, lds, gamma, beta);
  else if (af.mode == 1) { gamma = af.gb[c]; beta = af.gb[C + c]; }
  const RowAffine ra = row_affine(af, C, c, gamma, beta);
  const float* xr = x + row * T;
  float s = 0.0f;
  for (int64_t i = g; i < T; i += kRowBlock) s += xr[i];
  const float mean = group_sum<kRowBlock>(s, lds) / static_cast<float>(T);
  float q = 0.0f;
  for (int64_t i = g; i < T; i += kRowBlock) {
    const float d = xr[i] - mean;
    q += d * d;
  }
  const float var = group_sum<kRowBlock>(q, lds) / static_cast<float>(T);
  const float den = sqrtf(var + eps);
  float* orow = out + row * T;
  for (int64_t i = g; i < T; i += kRowBlock) orow[i] = apply_affine<false>((xr[i] - mean) / den, ra, af);
}

// acc = 0; acc += part[b] for b in order (numpy's outer loop over
// 8192-blocks), by one whole wave: the lanes load 64 partials at once
// (device-coherent loads: other blocks wrote them), then the sum walks
// them in order through readlane.  Every lane returns it.
__device__ __forceinline__ float np_fold(float* part, int nblk) {
  const int lane = threadIdx.x & 63;
  float acc = 0.0f;
  for (int b0 = 0; b0 < nblk; b0 += 64) {
    const float v = b0 + lane < nblk ? __hip_atomic_load(part + b0 + lane, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT)
                                     : 0.0f;
    const int m = nblk - b0 < 64 ? nblk - b0 : 64;
    for (int j = 0; j < m; ++j)
      acc += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
  }
  return acc;
}

// A row of T elements of a flat [rows, T] tensor, cut where the flat index
// row * T + i is a multiple of 4: hh head elements, nv groups of four from
// i = hh (there a float row takes 16-byte and a byte row 4-byte accesses,
// given bases so aligned), and the tail from hh + 4 nv.  edge() gives the
// head and tail elements, at most three each, to threads 0-7 of the row's
// first block.
struct RowSplit {
  int64_t hh, nv, T;
  __device__ __forceinline__ bool edge(int64_t& i) const {
    if (blockIdx.x != 0 || threadIdx.x >= 8) return false;
    const int t = static_cast<int>(threadIdx.x);
    i = t < 4 ? t : hh + 4 * nv + (t - 4);
    return t < 4 ? i < hh : i < T;
  }
};
__device__ __forceinline__ RowSplit row_split(int64_t row, int64_t T) {
  const int64_t hh = std::min<int64_t>(T, (4 - (row * T) % 4) % 4);
  return RowSplit{hh, (T - hh) / 4, T};
}

// Applies y = affine((x - mean) / den) with per-row (mean, den) =
// stats[row] from the numpy-order statistics passes below (long rows).
__global__ void __launch_bounds__(kRowBlock) instnorm_apply(float* __restrict__ out,
                                                            const float* __restrict__ x,
                                                            const float2* __restrict__ stats,
                                                            int64_t C, int64_t T, Affine af,
                                                            int vec) {
  const int64_t row = blockIdx.y;
  const int64_t c = row % C;
  float gamma = 0.0f, beta = 0.0f;
  if (af.mode == 1) { gamma = af.gb[c]; beta = af.gb[C + c]; }
  const RowAffine ra = row_affine(af, C, c, gamma, beta);
  const float2 st = stats[row];  // (mean, den)
  const KkDivisor dden = kk_divisor(st.y);
  const float* xr = x + row * T;
  float* orow = out + row * T;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t i0 = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (vec) {
    const RowSplit rsp = row_split(row, T);
    // (cached loads: the statistics pass before this one read the row, and
    // part of it is still in the last-level cache -- a second read of a
    // 208 MB tensor runs at 6.3 TB/s, 5.6 with non-temporal loads)
    for (int64_t k = i0; k < rsp.nv; k += stride) {
      const int64_t i = rsp.hh + 4 * k;
      const float4 v = *reinterpret_cast<const float4*>(xr + i);
      const float4 q = kk_div4(make_float4(v.x - st.x, v.y - st.x, v.z - st.x, v.w - st.x), dden);
      st_stream4(orow + i, make_float4(apply_affine(q.x, ra, af), apply_affine(q.y, ra, af),
                                       apply_affine(q.z, ra, af), apply_affine(q.w, ra, af)));
    }
    int64_t i;
    if (rsp.edge(i))
      st_stream(orow + i, apply_affine((xr[i] - st.x) / st.y, ra, af));
  } else {
    for (int64_t i = i0; i < T; i += stride)
      st_stream(orow + i, apply_affine((xr[i] - st.x) / st.y, ra, af));
  }
}

// y recomputed exactly as above, then DynamicQuantizeLinear's byte: the
// float y never reaches memory.  The scale and zero point come from the
// npart (min, max) partials in mm, which every block folds (min and max do
// not depend on the order, so every block finds the same; block (0, 0)
// stores them: no fold launch), or with mm NULL from params[0] (dql_fold's
// launch, for more partials than a block folds).  only_if: the launch does
// nothing unless *only_if == epoch.  check: a y outside the folded (min,
// max) (params[1] with mm NULL) sets *check = epoch -- a value no earlier
// call leaves there, so nothing has to clear it first.  bmm: every block
// also stores the exact (min, max) of its y in bmm[row * gridDim.x +
// blockIdx.x], the partials a flagged call folds before quantising again.
__global__ void __launch_bounds__(kRowBlock) instnorm_quant(uint8_t* __restrict__ q,
                                                            const float* __restrict__ x,
                                                            const float2* __restrict__ stats,
                                                            const float2* __restrict__ params,
                                                            const float2* __restrict__ mm, int npart,
                                                            float* __restrict__ ysp,
                                                            uint8_t* __restrict__ yzp,
                                                            int64_t C, int64_t T, Affine af,
                                                            int vec, const int* __restrict__ only_if,
                                                            int* __restrict__ check, int epoch,
                                                            float2* __restrict__ bmm) {
  if (only_if && *only_if != epoch) return;
  __shared__ float2 wmm[kRowBlock / 64];
  __shared__ float4 pl;  // scale, zero point, and the (min, max) of y
  if (mm) {
    float lo = INFINITY, hi = -INFINITY;
    for (int i = threadIdx.x; i < npart; i += kRowBlock) {
      const float2 p = mm[i];
      lo = fminf(lo, p.x);
      hi = fmaxf(hi, p.y);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      lo = fminf(lo, __shfl_xor(lo, off, 64));
      hi = fmaxf(hi, __shfl_xor(hi, off, 64));
    }
    if ((threadIdx.x & 63) == 0) wmm[threadIdx.x >> 6] = make_float2(lo, hi);
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int w = 1; w < kRowBlock / 64; ++w) {
        lo = fminf(lo, wmm[w].x);
        hi = fmaxf(hi, wmm[w].y);
      }
      float sc;
      uint8_t zq;
      const float2 pz = dql_params(lo, hi, &sc, &zq);
      if (blockIdx.x == 0 && blockIdx.y == 0) {
        *ysp = sc;
        *yzp = zq;
      }
      pl = make_float4(pz.x, pz.y, lo, hi);
    }
  } else if (threadIdx.x == 0) {
    const float2 p0 = params[0];
    const float2 p1 = check ? params[1] : make_float2(-INFINITY, INFINITY);
    pl = make_float4(p0.x, p0.y, p1.x, p1.y);
  }
  __syncthreads();
  const int64_t row = blockIdx.y;
  const int64_t c = row % C;
  const RowAffine ra = row_affine(af, C, c, 0.0f, 0.0f);
  const float4 P = pl;
  const float2 st = stats[row], pz = make_float2(P.x, P.y);
  const KkDivisor dden = kk_divisor(st.y), dsc = kk_divisor(pz.x);
  const float2 lim = make_float2(P.z, P.w);
  const float* xr = x + row * T;
  uint8_t* qr = q + row * T;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t i0 = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  float lo = INFINITY, hi = -INFINITY;  // this thread's (min, max) of y
  if (vec) {
    const RowSplit rsp = row_split(row, T);
    for (int64_t k = i0; k < rsp.nv; k += stride) {
      const int64_t i = rsp.hh + 4 * k;
      const float4 v = *reinterpret_cast<const float4*>(xr + i);  // cached: as instnorm_apply
      const float4 q = kk_div4(make_float4(v.x - st.x, v.y - st.x, v.z - st.x, v.w - st.x), dden);
      const float y0 = apply_affine(q.x, ra, af);
      const float y1 = apply_affine(q.y, ra, af);
      const float y2 = apply_affine(q.z, ra, af);
      const float y3 = apply_affine(q.w, ra, af);
      lo = fminf(lo, fminf(fminf(y0, y1), fminf(y2, y3)));
      hi = fmaxf(hi, fmaxf(fmaxf(y0, y1), fmaxf(y2, y3)));
      const uint32_t w = dql_bytes4(make_float4(y0, y1, y2, y3), dsc, pz.y);
      // an ordinary store: the convolution that reads the bytes next finds
      // them in the last-level cache
      *reinterpret_cast<uint32_t*>(qr + i) = w;
    }
    int64_t i;
    if (rsp.edge(i)) {
      const float y = apply_affine((xr[i] - st.x) / st.y, ra, af);
      lo = fminf(lo, y);
      hi = fmaxf(hi, y);
      qr[i] = static_cast<uint8_t>(dql_byte(y, pz.x, pz.y));
    }
  } else {
    for (int64_t i = i0; i < T; i += stride) {
      const float y = apply_affine((xr[i] - st.x) / st.y, ra, af);
      lo = fminf(lo, y);
      hi = fmaxf(hi, y);
      qr[i] = static_cast<uint8_t>(dql_byte(y, pz.x, pz.y));
    }
  }
  if (check && (lo < lim.x || hi > lim.y)) *check = epoch;  // every writer stores the same value
  if (bmm) {  // (uniform: every thread of the block takes the barrier)
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      lo = fminf(lo, __shfl_xor(lo, off, 64));
      hi = fmaxf(hi, __shfl_xor(hi, off, 64));
    }
    if ((threadIdx.x & 63) == 0) wmm[threadIdx.x >> 6] = make_float2(lo, hi);
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int w = 1; w < kRowBlock / 64; ++w) {
        lo = fminf(lo, wmm[w].x);
        hi = fmaxf(hi, wmm[w].y);
      }
      bmm[row * gridDim.x + blockIdx.x] = make_float2(lo, hi);
    }
  }
}

// -------------------------------------------------------------- LayerNorm
struct LnArgs {
  const float* skip;       // [rows, cols] or NULL
  const float* skip_bias;  // [cols] or NULL
  const float* scale;      // [cols]
  const float* bias;       // [cols] or NULL
};

template <int GROUP, int NV, int VEC>
__global__ void __launch_bounds__(kRowBlock) layernorm_kernel(float* __restrict__ out,
                                                              const float* __restrict__ x,
                                                              int64_t rows, int64_t cols, float eps,
                                                              LnArgs la) {
  __shared__ float lds[4];
  const int RPB = blockDim.x / GROUP;  // 256 / GROUP, or 1 in 64-thread blocks
  const int g = threadIdx.x % GROUP;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / GROUP;
  if constexpr (GROUP == 64) {
    if (row >= rows) return;
  }
  float r[NV][VEC];
  load_row<GROUP, NV, VEC>(x + row * cols, cols, g, r);
  if (la.skip) {
    // SkipLayerNormalization: s = x + skip (+ bias), ref_runtime.py:605-608.
    float k[NV][VEC];
    load_row<GROUP, NV, VEC>(la.skip + row * cols, cols, g, k);
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int e = 0; e < VEC; ++e) r[j][e] = r[j][e] + k[j][e];
    if (la.skip_bias) {
      load_row<GROUP, NV, VEC, false>(la.skip_bias, cols, g, k);
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < VEC; ++e) r[j][e] = r[j][e] + k[j][e];
    }
  }
  // scale and bias are loaded before the statistics, so their latency
  // overlaps the row's instead of following the reductions
  float sc[NV][VEC], bi[NV][VEC];
  load_row<GROUP, NV, VEC, false>(la.scale, cols, g, sc);
  if (la.bias) load_row<GROUP, NV, VEC, false>(la.bias, cols, g, bi);
  float mean, var;
  row_stats<GROUP, NV, VEC, true>(r, cols, g, lds, mean, var);
  const float inv = 1.0f / sqrtf(var + eps);  // one division per row (rel 1e-4 bar)
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int e = 0; e < VEC; ++e) r[j][e] = (r[j][e] * inv) * sc[j][e];
  if (la.bias) {
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int e = 0; e < VEC; ++e) r[j][e] = r[j][e] + bi[j][e];
  }
  store_row<GROUP, NV, VEC>(out + row * cols, cols, g, r);
}

// LayerNorm (no skip input) over one row per wave, for rows of
// 64 (NV - 1) < cols / 4 <= 64 NV float4s ([256, 768]: three each): the
// row, scale and bias in registers, vectors 0 .. NV-2 whole for every lane
// (only the last one guarded), the two sums DPP moves within the wave, the
// statistics scaled by 1 / cols and normalised with the hardware reciprocal
// square root (within 1 ulp; LayerNorm is held to rel 1e-4), the output
// (d * inv) * scale + bias one multiply and one FMA per element.
template <int NV, bool BIAS>
__global__ void __launch_bounds__(64) layernorm_row_kernel(float* __restrict__ out,
                                                          const float* __restrict__ x, int cols,
                                                          float inv_c, float eps,
                                                          const float* __restrict__ scale,
                                                          const float* __restrict__ bias) {
  const int g = threadIdx.x;
  const int64_t row = blockIdx.x;
  const float* __restrict__ xr = x + row * cols;
  const bool tail = (NV - 1) * 64 + g < (cols >> 2);
  const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  float4 v[NV], sc[NV], bi[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int i = 4 * (j * 64 + g);
    const bool in = j < NV - 1 || tail;
    v[j] = in ? ld_stream4(xr + i) : z;
    sc[j] = in ? *reinterpret_cast<const float4*>(scale + i) : z;
    bi[j] = BIAS && in ? *reinterpret_cast<const float4*>(bias + i) : z;
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  const float mean = wave_sum_dpp(s) * inv_c;
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    v[j].x -= mean;
    v[j].y -= mean;
    v[j].z -= mean;
    v[j].w -= mean;
    float t = __builtin_fmaf(v[j].x, v[j].x, v[j].y * v[j].y);
    t = __builtin_fmaf(v[j].z, v[j].z, t);
    t = __builtin_fmaf(v[j].w, v[j].w, t);
    if (j < NV - 1 || tail) q += t;
  }
  const float inv = __builtin_amdgcn_rsqf(__builtin_fmaf(wave_sum_dpp(q), inv_c, eps));
  float* __restrict__ orow = out + row * cols;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const float4 y = make_float4(__builtin_fmaf(v[j].x * inv, sc[j].x, bi[j].x),
                                 __builtin_fmaf(v[j].y * inv, sc[j].y, bi[j].y),
                                 __builtin_fmaf(v[j].z * inv, sc[j].z, bi[j].z),
                                 __builtin_fmaf(v[j].w * inv, sc[j].w, bi[j].w));
    if (j < NV - 1 || tail) st_stream4(orow + 4 * (j * 64 + g), y);
  }
}

__global__ void __launch_bounds__(kRowBlock) layernorm_long_kernel(float* __restrict__ out,
                                                                   const float* __restrict__ x,
                                                                   int64_t cols, float eps,
                                                                   LnArgs la) {
  __shared__ float lds[4];
  const int g = threadIdx.x;
  const int64_t row = blockIdx.x;
  const float* xr = x + row * cols;
  const float* kr = la.skip ? la.skip + row * cols : nullptr;
  auto val = [&](int64_t i) {
    float v = xr[i];
    if (kr) {
      v = v + kr[i];
      if (la.skip_bias) v = v + la.skip_bias[i];
    }
    return v;
  };
  float s = 0.0f;
  for (int64_t i = g; i < cols; i += kRowBlock) s += val(i);
  const float mean = group_sum<kRowBlock>(s, lds) / static_cast<float>(cols);
  float q = 0.0f;
  for (int64_t i = g; i < cols; i += kRowBlock) {
    const float d = val(i) - mean;
    q += d * d;
  }
  const float var = group_sum<kRowBlock>(q, lds) / static_cast<float>(cols);
  const float den = sqrtf(var + eps);
  float* orow = out + row * cols;
  for (int64_t i = g; i < cols; i += kRowBlock) {
    float v = ((val(i) - mean) / den) * la.scale[i];
    if (la.bias) v = v + la.bias[i];
    orow[i] = v;
  }
}

// ---------------------------------------------------------------- Softmax
template <int GROUP, int NV, int VEC>
__global__ void __launch_bounds__(kRowBlock) softmax_kernel(float* __restrict__ out,
                                                            const float* __restrict__ x,
                                                            int64_t rows, int64_t cols) {
  __shared__ float lds[4];
  const int RPB = blockDim.x / GROUP;  // 256 / GROUP, or 1 in 64-thread blocks
  const int g = threadIdx.x % GROUP;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / GROUP;
  if constexpr (GROUP == 64) {
    if (row >= rows) return;
  }
  float r[NV][VEC];
  load_row<GROUP, NV, VEC>(x + row * cols, cols, g, r);
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t base = (static_cast<int64_t>(j) * GROUP + g) * VEC;
#pragma unroll
    for (int e = 0; e < VEC; ++e)
      if (base + e < cols) m = fmaxf(m, r[j][e]);
  }
  m = group_max<GROUP, true>(m, lds);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t base = (static_cast<int64_t>(j) * GROUP + g) * VEC;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float v = kk_exp_neg(r[j][e] - m);  // (x - max <= 0; held to rel 1e-4)
      r[j][e] = v;
      if (base + e < cols) s += v;
    }
  }
  // the hardware reciprocal, once per row (within 1 ulp; rel 1e-4 bar)
  const float inv = __builtin_amdgcn_rcpf(group_sum<GROUP, true>(s, lds));
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int e = 0; e < VEC; ++e) r[j][e] = r[j][e] * inv;
  store_row<GROUP, NV, VEC>(out + row * cols, cols, g, r);
}

// Softmax / reduce along an axis with inner extent > 1: one thread per
// (outer, inner) column walks the axis (coalesced across inner).
__global__ void softmax_cols_kernel(float* __restrict__ out, const float* __restrict__ x,
                                    int64_t outer, int64_t dim, int64_t inner) {
  const int64_t n = outer * inner;
  for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < n;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t o = t / inner, i = t % inner;
    const float* xc = x + o * dim * inner + i;
    float* oc = out + o * dim * inner + i;
    float m = -INFINITY;
    for (int64_t d = 0; d < dim; ++d) m = fmaxf(m, xc[d * inner]);
    double s = 0.0;
    for (int64_t d = 0; d < dim; ++d) s += expf(xc[d * inner] - m);
    const float sf = static_cast<float>(s);
    for (int64_t d = 0; d < dim; ++d) oc[d * inner] = expf(xc[d * inner] - m) / sf;
  }
}

// ------------------------------------------------------------- reductions
template <int GROUP, int NV, int VEC>
__global__ void __launch_bounds__(kRowBlock) reduce_rows_kernel(float* __restrict__ out,
                                                                const float* __restrict__ x,
                                                                int64_t rows, int64_t cols, int op) {
  __shared__ float lds[4];
  const int RPB = blockDim.x / GROUP;  // 256 / GROUP, or 1 in 64-thread blocks
  const int g = threadIdx.x % GROUP;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / GROUP;
  if constexpr (GROUP == 64) {
    if (row >= rows) return;
  }
  float r[NV][VEC];
  load_row<GROUP, NV, VEC>(x + row * cols, cols, g, r);
  float v;
  if (op == KK_REDUCE_MAX) {
    float m = -INFINITY;
    bool nan = false;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t base = (static_cast<int64_t>(j) * GROUP + g) * VEC;
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        if (base + e < cols) { nan |= __builtin_isnan(r[j][e]); m = fmaxf(m, r[j][e]); }
    }
    m = group_max<GROUP>(m, lds);
    const float anynan = group_max<GROUP>(nan ? 1.0f : 0.0f, lds);
    v = anynan > 0.0f ? NAN : m;
  } else {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int e = 0; e < VEC; ++e) s += r[j][e];
    s = group_sum<GROUP>(s, lds);
    v = op == KK_REDUCE_MEAN ? s / static_cast<float>(cols) : s;
  }
  if (g == 0) out[row] = v;
}

// ------------------------------------------------- numpy-order summation
// numpy reduces a float32 row (np.sum / np.mean over a contiguous axis, as
// every ReduceMean/ReduceSum of the graph and the InstanceNorm statistics
// do) as
//   acc = 0; for each 8192-element block of the row, in order: acc += pw(block)
// where 8192 is the ufunc buffer size and pw is numpy's pairwise_sum
// (numpy/_core/src/umath/loops_utils.h.src):
//   n < 8:     sequential from 0
//   n <= 128:  eight strided accumulators r[j] += a[i + j], combined as
//              ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7)), then the
//              n % 8 tail added in order
//   else:      pw(a, n2) + pw(a + n2, n - n2), n2 = n / 2 rounded down to a
//              multiple of 8.
// The kernels below evaluate exactly this tree, so their sums and means
// carry numpy's roundings bit for bit.  A 512-thread block owns one 8192
// block: eight lanes per leaf (a full block has 64 leaves of 128 in a
// balanced tree, reduced with shuffles and an 8-entry LDS step); a partial
// block (a row's tail) enumerates its leaves and evaluates its tree in one
// thread.  Rows sit in LDS padded by 8 floats per 128, which puts the 64
// lanes of a leaf step on 64 distinct banks.
constexpr int kNpBlock = 8192;
constexpr int kNpLeaf = 128;
constexpr int kNpThreads = 512;
constexpr int kNpMaxLeaves = 72;  // at most 65 leaves for n <= 8192
constexpr int kNpDepth = 8;       // the recursion is at most 7 deep for n <= 8192

__device__ __forceinline__ int np_pad(int e) { return e + 8 * (e >> 7); }

struct NpScratch {
  int lo[kNpMaxLeaves], n[kNpMaxLeaves];
  float sum[kNpMaxLeaves];
  float wave[kNpThreads / 64];
  float wmin[kNpThreads / 64], wmax[kNpThreads / 64];
  int count;
  float total;
};

template <int D>
__device__ void np_leaves(int lo, int n, int& k, NpScratch& S) {
  if constexpr (D == 0) {
    S.lo[k] = lo; S.n[k] = n; ++k;
  } else {
    if (n <= kNpLeaf) { S.lo[k] = lo; S.n[k] = n; ++k; return; }
    int n2 = n / 2;
    n2 -= n2 % 8;
    np_leaves<D - 1>(lo, n2, k, S);
    np_leaves<D - 1>(lo + n2, n - n2, k, S);
  }
}

template <int D>
__device__ float np_tree(int n, int& k, const NpScratch& S) {
  if constexpr (D == 0) {
    return S.sum[k++];
  } else {
    if (n <= kNpLeaf) return S.sum[k++];
    int n2 = n / 2;
    n2 -= n2 % 8;
    const float a = np_tree<D - 1>(n2, k, S);
    const float b = np_tree<D - 1>(n - n2, k, S);
    return a + b;
  }
}

// numpy's pairwise sum of f(i), i in [0, m), 1 <= m <= 8192, by a whole
// 512-thread block; every thread returns the sum.  f reads LDS or computes.
template <class F>
__device__ __forceinline__ float np_block_sum(F f, int m, NpScratch& S) {
  const int q = threadIdx.x >> 3, j = threadIdx.x & 7;
  if (m == kNpBlock) {
    float r = f(q * kNpLeaf + j);
#pragma unroll
    for (int i = 8; i < kNpLeaf; i += 8) r += f(q * kNpLeaf + i + j);
    r += __shfl_xor(r, 1, 64);   // leaf q: ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7))
    r += __shfl_xor(r, 2, 64);
    r += __shfl_xor(r, 4, 64);
    r += __shfl_xor(r, 8, 64);   // leaves 8w .. 8w+7 of wave w, balanced
    r += __shfl_xor(r, 16, 64);
    r += __shfl_xor(r, 32, 64);
    if ((threadIdx.x & 63) == 0) S.wave[threadIdx.x >> 6] = r;
    __syncthreads();
    const float s = ((S.wave[0] + S.wave[1]) + (S.wave[2] + S.wave[3])) +
                    ((S.wave[4] + S.wave[5]) + (S.wave[6] + S.wave[7]));
    __syncthreads();
    return s;
  }
  if (threadIdx.x == 0) {
    int k = 0;
    np_leaves<kNpDepth>(0, m, k, S);
    S.count = k;
  }
  __syncthreads();
  for (int base = 0; base < S.count; base += kNpThreads / 8) {
    const int leaf = base + q;
    if (leaf < S.count) {  // uniform over the leaf's eight lanes
      const int lo = S.lo[leaf], n = S.n[leaf];
      float res = 0.0f;
      if (n < 8) {
        if (j == 0)
          for (int i = 0; i < n; ++i) res += f(lo + i);
      } else {
        const int body = n - n % 8;
        float r = f(lo + j);
        for (int i = 8; i < body; i += 8) r += f(lo + i + j);
        r += __shfl_xor(r, 1, 64);
        r += __shfl_xor(r, 2, 64);
        r += __shfl_xor(r, 4, 64);
        res = r;
        if (j == 0)
          for (int i = body; i < n; ++i) res += f(lo + i);
      }
      if (j == 0) S.sum[leaf] = res;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int k = 0;
    S.total = np_tree<kNpDepth>(m, k, S);
  }
  __syncthreads();
  const float s = S.total;
  __syncthreads();
  return s;
}

// Loads elements [0, n) of `src` into the padded LDS row `dst`.
__device__ __forceinline__ void np_load_row(float* dst, const float* __restrict__ src, int64_t n,
                                            bool vec) {
  if (vec) {
    for (int64_t e = 4 * threadIdx.x; e < n; e += 4 * kNpThreads) {
      const float4 v = ld_stream4(src + e);
      *reinterpret_cast<float4*>(dst + np_pad(static_cast<int>(e))) = v;
    }
  } else {
    for (int64_t e = threadIdx.x; e < n; e += kNpThreads) dst[np_pad(static_cast<int>(e))] = ld_stream(src + e);
  }
}


// numpy's pairwise tree over a row's last, partial 8192-block of m
// elements (0 < m < 8192; nleaf = 0 when the row has none): its leaves
// (lo, n) in order, then its internal nodes level by level, node k =
// v[ca[k]] + v[cb[k]] over ids 0 .. nleaf-1 (the leaves) and nleaf + k (the
// nodes), each node's children in earlier levels; level l's nodes end at
// lev_end[l].  Built on the host: every row of a launch shares m.
constexpr int kTailMax = 72;
struct NpTail {
  int m, nleaf, nnode, nlev;
  uint16_t lo[kTailMax];
  uint8_t n[kTailMax];
  uint8_t ca[kTailMax], cb[kTailMax];
  uint8_t lev_end[kNpDepth];
};
// lo, n, ca and cb as 32-bit words (np_resident_kernel copies them as such)
constexpr int kPlanWords = 5 * kTailMax / 4;
static_assert(offsetof(NpTail, lo) % 4 == 0 && offsetof(NpTail, n) == offsetof(NpTail, lo) + 2 * kTailMax &&
                  offsetof(NpTail, ca) == offsetof(NpTail, n) + kTailMax &&
                  offsetof(NpTail, cb) == offsetof(NpTail, ca) + kTailMax && (5 * kTailMax) % 4 == 0,
              "the plan's arrays are contiguous 32-bit words");

// The plan in LDS (its lane-indexed reads would otherwise be memory loads)
// and the partial block's node values.
struct NpPlanLds {
  uint16_t lo[kTailMax];
  uint8_t n[kTailMax], ca[kTailMax], cb[kTailMax];
  float tv[2 * kTailMax];
};
__device__ __forceinline__ void np_plan_to_lds(const NpTail& tail, NpPlanLds& P) {
  if (threadIdx.x < kTailMax) {
    P.lo[threadIdx.x] = tail.lo[threadIdx.x];
    P.n[threadIdx.x] = tail.n[threadIdx.x];
    P.ca[threadIdx.x] = tail.ca[threadIdx.x];
    P.cb[threadIdx.x] = tail.cb[threadIdx.x];
  }
}

// numpy's pairwise sum of f(i), i in [0, tail.m), over the plan: eight lanes
// a leaf with all sixteen terms of an accumulator read at once, then wave 0
// walks the tree a level at a time (LDS accesses of one wave take effect in
// order).  By the whole block (plan in P, after a barrier); every thread
// returns the sum.
template <class F>
__device__ float np_tail_sum(F f, const NpTail& tail, NpPlanLds& P, NpScratch& S) {
  const int j = threadIdx.x & 7, m = tail.m;
  for (int leaf = threadIdx.x >> 3; leaf < tail.nleaf; leaf += blockDim.x / 8) {
    const int lo = P.lo[leaf], n = P.n[leaf];  // uniform over the leaf's lanes
    const int body = n - n % 8;
    float res = 0.0f;
    if (body) {
      float term[kNpLeaf / 8];
#pragma unroll
      for (int k = 0; k < kNpLeaf / 8; ++k) term[k] = f(min(lo + 8 * k + j, m - 1));
      float q = term[0];
#pragma unroll
      for (int k = 1; k < kNpLeaf / 8; ++k)
        if (8 * k < body) q += term[k];
      q += dpp_move<0xB1, 0xF>(q, 0.0f);   // lane pairs (xor 1)
      q += dpp_move<0x4E, 0xF>(q, 0.0f);   // quads (xor 2)
      q += dpp_move<0x141, 0xF>(q, 0.0f);  // eights (row half mirror: xor 4 once quads agree)
      res = q;
    }
    if (j == 0) {  // the n % 8 last terms (all of them when n < 8), in order
      float xt[7];
#pragma unroll
      for (int i = 0; i < 7; ++i) xt[i] = f(min(lo + body + i, m - 1));
#pragma unroll
      for (int i = 0; i < 7; ++i)
        if (body + i < n) res += xt[i];
      P.tv[leaf] = res;
    }
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    for (int l = 0; l < tail.nlev; ++l) {
      const int k = (l ? tail.lev_end[l - 1] : 0) + static_cast<int>(threadIdx.x);
      if (k < tail.lev_end[l]) P.tv[tail.nleaf + k] = P.tv[P.ca[k]] + P.tv[P.cb[k]];
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
    if (threadIdx.x == 0) S.total = P.tv[tail.nnode ? tail.nleaf + tail.nnode - 1 : 0];
  }
  __syncthreads();
  const float s = S.total;
  __syncthreads();
  return s;
}

// numpy-order sum of the padded LDS row (n elements) of f(x), acc from 0.
// The partial block (if any) over the plan, whose m is n % 8192.
template <class F>
__device__ float np_row_sum(const float* row, int n, F f, NpScratch& S, const NpTail& tail,
                            NpPlanLds& P) {
  float acc = 0.0f;
  for (int b0 = 0; b0 < n; b0 += kNpBlock) {
    const auto g = [&](int i) { return f(row[np_pad(b0 + i)]); };
    acc += n - b0 < kNpBlock ? np_tail_sum(g, tail, P, S) : np_block_sum(g, kNpBlock, S);
  }
  return acc;
}

// Rows of at most 2 x 8192 elements, one block per row, the row in LDS.
//   mode 0: out[row] = sum       mode 1: out[row] = sum / n
//   mode 2: instance norm of the row with the affine `af` into out
__global__ void __launch_bounds__(kNpThreads) np_rows_kernel(float* __restrict__ out,
                                                             const float* __restrict__ x,
                                                             int64_t C, int n, int mode,
                                                             float eps, Affine af, int vec,
                                                             float2* __restrict__ stats,
                                                             float2* __restrict__ mm,
                                                             NpTail tail) {
  extern __shared__ __align__(16) float np_lds[];
  __shared__ NpScratch S;
  __shared__ NpPlanLds P;
  const int64_t row = blockIdx.x;
  const float* xr = x + row * n;
  np_plan_to_lds(tail, P);
  np_load_row(np_lds, xr, n, vec);
  __syncthreads();
  const float sum = np_row_sum(np_lds, n, [](float v) { return v; }, S, tail, P);
  if (mode < 2) {
    if (threadIdx.x == 0) out[row] = mode == 1 ? sum / static_cast<float>(n) : sum;
    return;
  }
  const float mean = sum / static_cast<float>(n);
  const float sq = np_row_sum(np_lds, n, [mean](float v) { const float d = v - mean; return d * d; },
                              S, tail, P);
  const float den = sqrtf(sq / static_cast<float>(n) + eps);
  const int64_t c = row % C;
  float gamma = 0.0f, beta = 0.0f;
  if (af.mode == 1) { gamma = af.gb[c]; beta = af.gb[C + c]; }
  const RowAffine ra = row_affine(af, C, c, gamma, beta);
  const KkDivisor dden = kk_divisor(den);
  if (mode == 3) {  // no output: (mean, den) and the (min, max) of the row's results
    float lo = INFINITY, hi = -INFINITY;
    for (int e = threadIdx.x; e < n; e += kNpThreads) {
      const float y = apply_affine(kk_div(np_lds[np_pad(e)] - mean, dden), ra, af);
      lo = fminf(lo, y);
      hi = fmaxf(hi, y);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      lo = fminf(lo, __shfl_xor(lo, off, 64));
      hi = fmaxf(hi, __shfl_xor(hi, off, 64));
    }
    __shared__ float2 wmm[kNpThreads / 64];
    if ((threadIdx.x & 63) == 0) wmm[threadIdx.x >> 6] = make_float2(lo, hi);
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int w = 1; w < kNpThreads / 64; ++w) {
        lo = fminf(lo, wmm[w].x);
        hi = fmaxf(hi, wmm[w].y);
      }
      stats[row] = make_float2(mean, den);
      mm[row] = make_float2(lo, hi);
    }
    return;
  }
  float* orow = out + row * n;
  if (vec) {
    for (int e = 4 * threadIdx.x; e < n; e += 4 * kNpThreads) {
      const float4 v = *reinterpret_cast<const float4*>(np_lds + np_pad(e));
      const float4 q = kk_div4(make_float4(v.x - mean, v.y - mean, v.z - mean, v.w - mean), dden);
      st_stream4(orow + e, make_float4(apply_affine(q.x, ra, af), apply_affine(q.y, ra, af),
                                       apply_affine(q.z, ra, af), apply_affine(q.w, ra, af)));
    }
  } else {
    for (int e = threadIdx.x; e < n; e += kNpThreads)
      st_stream(orow + e, apply_affine((np_lds[np_pad(e)] - mean) / den, ra, af));
  }
}

// The (min, max) of wave-spread values lo, hi over the whole block: each
// wave's lane 0 leaves its pair in S.wmin / S.wmax (read after a barrier).
__device__ __forceinline__ void np_wave_minmax(float lo, float hi, NpScratch& S) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, off, 64));
    hi = fmaxf(hi, __shfl_xor(hi, off, 64));
  }
  if ((threadIdx.x & 63) == 0) {
    S.wmin[threadIdx.x >> 6] = lo;
    S.wmax[threadIdx.x >> 6] = hi;
  }
}

// Long rows: block (b, row) computes pw of 8192-block b of f(x) into
// part[row][b]; f is x (mode 0) or (x - mean)^2 (mode 1, mean in
// stats[row].x).  The last block of a row to finish (counted in
// cnt[row * cstride], which it resets) folds the row's partials in block order, acc = 0;
// acc += part[b] (numpy's loop over 8192-blocks), and writes
//   mode 0: red_out[row] = acc (or acc / T when red_mean), or without
//           red_out stats[row].x = acc / T (ReduceMean's division)
//   mode 1: stats[row].y = sqrt(acc / T + eps)
// Once its block sum is formed only wave 0 stays: the other waves leave
// while it publishes the partial and counts.
// With xmm, mode 0 also leaves the block's (min, max) of x in
// xmm[row * nblk + b]; with mm, mode 1's last block folds the row's xmm
// into (xmin, xmax) and writes mm[row] = the (min, max) of
// y = affine((x - mean) / den) at those two points: the row's (min, max)
// of y whenever y is monotonic in x.
__global__ void __launch_bounds__(kNpThreads) np_blocks_kernel(
    float* __restrict__ part, const float* __restrict__ x, int64_t T, int nblk, int mode,
    float2* __restrict__ stats, int* __restrict__ cnt, int cstride, float* __restrict__ red_out,
    int red_mean, float eps, float2* __restrict__ xmm, float2* __restrict__ mm, int64_t C,
    Affine af, NpTail tail, const float* __restrict__ leaves, int64_t nleaf) {
  __shared__ NpScratch S;
  const int64_t row = blockIdx.y;
  cnt += row * cstride;  // counters spaced apart: the rows' atomics do not share a line
  const int b = blockIdx.x;
  const int64_t lo = static_cast<int64_t>(b) * kNpBlock;
  const int m = static_cast<int>(T - lo < kNpBlock ? T - lo : kNpBlock);
  const float mean = mode == 1 ? stats[row].x : 0.0f;
  auto f = [mode, mean](float e) {
    if (mode == 0) return e;
    const float d = e - mean;
    return d * d;
  };
  const float* xb = x + row * T + lo;
  // xmm: the (min, max) of x of each block, formed in the second pass (the
  // first may take its sums from leaves and not read x) and read by that
  // pass's last block of the row: stored and loaded at the device-coherent
  // level, as the partials are
  const bool want_xmm = xmm && mode == 1;
  float s;
  if (m == kNpBlock && leaves && mode == 0) {
    // the 64 leaf sums of this block, formed by the producer of x in the
    // same order (kk_conv_integer_scaled_qbias_packed_leaves): the balanced
    // tree of the full-block path below
    if (threadIdx.x >= 64) return;
    float r = leaves[row * nleaf + static_cast<int64_t>(b) * 64 + threadIdx.x];
    r += __shfl_xor(r, 1, 64);
    r += __shfl_xor(r, 2, 64);
    r += __shfl_xor(r, 4, 64);
    r += __shfl_xor(r, 8, 64);
    r += __shfl_xor(r, 16, 64);
    r += __shfl_xor(r, 32, 64);
    s = r;
  } else if (m == kNpBlock) {
    // A whole block straight from memory into the summation order: lane j
    // of leaf q (eight lanes per 128-element leaf) holds elements
    // q*128 + 8k + j, k = 0..15, its accumulator's terms in order.  (Staging
    // the block through LDS with 16-byte loads measured slower.)
    const int q = threadIdx.x >> 3, j = threadIdx.x & 7;
    float v[kNpLeaf / 8];
#pragma unroll
    for (int k = 0; k < kNpLeaf / 8; ++k) v[k] = xb[q * kNpLeaf + 8 * k + j];
    float r = f(v[0]);
#pragma unroll
    for (int k = 1; k < kNpLeaf / 8; ++k) r += f(v[k]);
    r += __shfl_xor(r, 1, 64);   // leaf q: ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7))
    r += __shfl_xor(r, 2, 64);
    r += __shfl_xor(r, 4, 64);
    r += __shfl_xor(r, 8, 64);   // leaves 8w .. 8w+7 of wave w, balanced
    r += __shfl_xor(r, 16, 64);
    r += __shfl_xor(r, 32, 64);
    if ((threadIdx.x & 63) == 0) S.wave[threadIdx.x >> 6] = r;
    if (want_xmm) {
      float lo = v[0], hi = v[0];
#pragma unroll
      for (int k = 1; k < kNpLeaf / 8; ++k) {
        lo = fminf(lo, v[k]);
        hi = fmaxf(hi, v[k]);
      }
      np_wave_minmax(lo, hi, S);
    }
    __syncthreads();
    if (threadIdx.x >= 64) return;
    s = ((S.wave[0] + S.wave[1]) + (S.wave[2] + S.wave[3])) +
        ((S.wave[4] + S.wave[5]) + (S.wave[6] + S.wave[7]));
  } else {
    // the row's last, partial block: its leaves and tree from the
    // host-built plan (every row of the launch shares m), eight lanes a
    // leaf with all sixteen terms of an accumulator loaded at once (a loop
    // of dependent loads, one memory round trip a term, cost ~10 us a
    // launch at [1,128,430800]), then wave 0's walk of the tree
    __shared__ uint16_t p_lo[kTailMax];
    __shared__ uint8_t p_n[kTailMax], p_ca[kTailMax], p_cb[kTailMax];
    __shared__ float tv[2 * kTailMax];
    if (threadIdx.x < kTailMax) {
      p_lo[threadIdx.x] = tail.lo[threadIdx.x];
      p_n[threadIdx.x] = tail.n[threadIdx.x];
      p_ca[threadIdx.x] = tail.ca[threadIdx.x];
      p_cb[threadIdx.x] = tail.cb[threadIdx.x];
    }
    __syncthreads();
    const int j = threadIdx.x & 7;
    float lo_x = INFINITY, hi_x = -INFINITY;
    for (int leaf = threadIdx.x >> 3; leaf < tail.nleaf; leaf += kNpThreads / 8) {
      const int lo = p_lo[leaf], n = p_n[leaf];  // uniform over the leaf's lanes
      const int body = n - n % 8;
      float xv[kNpLeaf / 8], xt[7];
#pragma unroll
      for (int k = 0; k < kNpLeaf / 8; ++k) xv[k] = xb[min(lo + 8 * k + j, m - 1)];
#pragma unroll
      for (int i = 0; i < 7; ++i) xt[i] = xb[min(lo + body + i, m - 1)];
      float res = 0.0f;
      if (body) {
        float q = f(xv[0]);
#pragma unroll
        for (int k = 1; k < kNpLeaf / 8; ++k)
          if (8 * k < body) q += f(xv[k]);
        q += dpp_move<0xB1, 0xF>(q, 0.0f);   // lane pairs (xor 1)
        q += dpp_move<0x4E, 0xF>(q, 0.0f);   // quads (xor 2)
        q += dpp_move<0x141, 0xF>(q, 0.0f);  // eights (row half mirror: xor 4 once quads agree)
        res = q;
#pragma unroll
        for (int k = 0; k < kNpLeaf / 8; ++k)
          if (8 * k < body) {
            lo_x = fminf(lo_x, xv[k]);
            hi_x = fmaxf(hi_x, xv[k]);
          }
      }
      if (j == 0) {  // the leaf's n % 8 last terms (all of it when n < 8), in order
#pragma unroll
        for (int i = 0; i < 7; ++i)
          if (body + i < n) {
            res += f(xt[i]);
            lo_x = fminf(lo_x, xt[i]);
            hi_x = fmaxf(hi_x, xt[i]);
          }
        tv[leaf] = res;
      }
    }
    if (want_xmm) np_wave_minmax(lo_x, hi_x, S);
    __syncthreads();
    if (threadIdx.x >= 64) return;
    for (int l = 0; l < tail.nlev; ++l) {  // wave 0: the tree, a level at a time
      const int k = (l ? tail.lev_end[l - 1] : 0) + static_cast<int>(threadIdx.x);
      if (k < tail.lev_end[l]) tv[tail.nleaf + k] = tv[p_ca[k]] + tv[p_cb[k]];
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
    s = tv[tail.nnode ? tail.nleaf + tail.nnode - 1 : 0];
  }
  if (want_xmm && threadIdx.x == 0) {
    float lo = S.wmin[0], hi = S.wmax[0];
    for (int w = 1; w < kNpThreads / 64; ++w) {
      lo = fminf(lo, S.wmin[w]);
      hi = fmaxf(hi, S.wmax[w]);
    }
    __hip_atomic_store(reinterpret_cast<uint64_t*>(xmm) + row * nblk + b,
                       __builtin_bit_cast(uint64_t, make_float2(lo, hi)), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  // wave 0: the partial goes to the device-coherent level (an agent-scope
  // store writes through this XCD's L2) and has landed before the count
  // moves: vmcnt(0) waits for the store's acknowledgement, and the compiler
  // fence keeps the compiler from moving either access across the other.  A
  // release fence would order the same two accesses by writing back this
  // XCD's whole L2 from every block (7x slower).
  int last = 0;
  if (threadIdx.x == 0) {
    __hip_atomic_store(part + row * nblk + b, s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nblk - 1;
  }
  if (__shfl(last, 0, 64)) {
    // the row's last block: an agent-scope acquire orders its reads of the
    // other blocks' partials after the count it saw (once per row)
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const float acc = np_fold(part + row * nblk, nblk);
    const float n = static_cast<float>(T);
    if (mode == 1 && mm) {  // the row's (xmin, xmax), from its blocks' xmm
      float lo = INFINITY, hi = -INFINITY;
      for (int i = threadIdx.x; i < nblk; i += 64) {
        const float2 p = __builtin_bit_cast(
            float2, __hip_atomic_load(reinterpret_cast<const uint64_t*>(xmm) + row * nblk + i,
                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        lo = fminf(lo, p.x);
        hi = fmaxf(hi, p.y);
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        lo = fminf(lo, __shfl_xor(lo, off, 64));
        hi = fmaxf(hi, __shfl_xor(hi, off, 64));
      }
      // the whole wave evaluates y (even lanes at xmin, odd at xmax)
      const float den = sqrtf(acc / n + eps);
      const int64_t c = row % C;
      float gamma = 0.0f, beta = 0.0f;
      if (af.mode == 1) { gamma = af.gb[c]; beta = af.gb[C + c]; }
      const RowAffine ra = row_affine(af, C, c, gamma, beta);
      const float y = apply_affine(((threadIdx.x & 1 ? hi : lo) - mean) / den, ra, af);
      const float y1 = __shfl_xor(y, 1, 64);
      if (threadIdx.x == 0) mm[row] = make_float2(fminf(y, y1), fmaxf(y, y1));
    }
    if (threadIdx.x == 0) {
      if (mode == 1) stats[row].y = sqrtf(acc / n + eps);
      else if (red_out) red_out[row] = red_mean ? acc / n : acc;
      else stats[row].x = acc / n;
      *cnt = 0;
    }
  }
}

// ------------------------------------- instance norm, row in registers
struct ResArgs {
  float* out;     // MODE 0: y = affine((x - mean) / den), no snake
  const float* x;
  float2* stats;  // MODE 2: (mean, den) per row
  float2* mm;     // MODE 2: (min, max) of y at the row's x extremes
  int64_t C, T;
  float eps;
  int stage_off;  // floats from the LDS base to the waves' stages
  int delay;      // MODE 0: the delayed half's wait, in 100 MHz clock ticks (0: none)
  Affine af;
  NpTail tail;
};

// Instance norm over rows of NB whole 8192-blocks and a partial one
// (15000 < T < 9 * 8192, T % 4 == 0; the decoder's [1,256,71800]), one
// workgroup of 128 NB threads per row, x read once.  Wave w holds the 4096
// floats (32 numpy leaves of 128) from 8192 (w / 2) + 4096 (w % 2) as
// sixteen float4s a lane in load order, k = 0..15 at 256 k + 4 lane: each
// load and each store of the wave is one contiguous 1 KB (holding each
// leaf's eight accumulators in a lane pair instead, 32-byte pieces, halved
// the read rate).  For a statistic the wave passes its leaves through its
// own LDS stage eight at a time (leaf pitch 136 floats: the 64 lanes'
// reads fall on distinct banks), where lane 8 q + j sums accumulator j of
// leaf q over its sixteen terms in order; three shuffles make the leaf
// ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7)), three more the
// balanced tree of the eight leaves, and ((c0 + c1) + (c2 + c3)) the
// wave's 32.  The block's two halves meet in LDS.  The partial block waits
// in LDS (padded as in np_rows_kernel) for eight lanes a leaf and wave 0's
// walk of its tree.  Both statistics are taken from registers, then
//   MODE 0: y is written from registers (no snake: sinf's slow path would
//           spill the held row);
//   MODE 2: nothing is written but stats[row] and mm[row] = the (min, max)
//           of y at the row's x extremes (for DynamicQuantizeLinear; x is
//           read with cached loads, for the quantising pass after it).
// The division by den is kk_div4's, bit-identical to the division.
template <int NB, int MODE>
__global__ void __launch_bounds__(128 * NB) np_resident_kernel(ResArgs A) {
  constexpr int NT = 128 * NB;
  constexpr int TPT = (kNpBlock / 4 + NT - 1) / NT;  // partial-block float4s a thread
  constexpr int kPitch = kNpLeaf + 8;
  extern __shared__ __align__(16) float res_lds[];  // the partial block, padded; the waves' stages
  __shared__ float ws[NT / 64];
  __shared__ float tv[2 * kTailMax];
  __shared__ float2 wmm[NT / 64];
  __shared__ float bc[4];
  // the tree plan (lo, n, ca, cb as laid out in NpTail)
  __shared__ uint32_t plan_w[kPlanWords];
  const uint16_t* const p_lo = reinterpret_cast<const uint16_t*>(plan_w);
  const uint8_t* const p_n = reinterpret_cast<const uint8_t*>(plan_w) + 2 * kTailMax;
  const uint8_t* const p_ca = p_n + kTailMax;
  const uint8_t* const p_cb = p_ca + kTailMax;
  float* const res_tail = res_lds;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t row = blockIdx.x;
  // MODE 0 with one block per CU: each block loads its row, reduces it and
  // stores it, so with every block in step HBM idles while they reduce and
  // no store overlaps a load.  Alternate groups of eight blocks (one a
  // XCD) start their loads A.delay ticks later -- about what the other
  // half's loads take -- so their loads overlap the first half's
  // statistics and stores.  The wait ends on the clock alone.
  if (MODE == 0 && A.delay && ((blockIdx.x >> 3) & 1)) {
    const uint64_t until = __builtin_amdgcn_s_memrealtime() + static_cast<uint64_t>(A.delay);
    while (__builtin_amdgcn_s_memrealtime() < until) __builtin_amdgcn_s_sleep(4);
  }
  const float* xr = A.x + row * A.T;
  const int m = A.tail.m, nleaf = A.tail.nleaf;
  // the partial block (buffer loads: past m they return zeros), the tree
  // plan, then the sixteen whole-block vectors
  const float* xt = xr + NB * kNpBlock;
  const auto rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(xt), 0, 4 * m, 0x00020000);
  float4 u[TPT];
#pragma unroll
  for (int i = 0; i < TPT; ++i) {
    const kk_f4v r = __builtin_bit_cast(
        kk_f4v, __builtin_amdgcn_raw_buffer_load_b128(rsrc, 16 * (t + i * NT), 0, 0));
    u[i] = make_float4(r.x, r.y, r.z, r.w);
  }
  if (t == NT - 64) {
    // the tree plan into LDS (its lane-indexed reads would otherwise be
    // memory loads each time), one lane: uniform reads of the kernel
    // argument are scalar loads, which wait on their own counter and not on
    // the row's loads
    const uint32_t* const src = reinterpret_cast<const uint32_t*>(A.tail.lo);
#pragma unroll
    for (int q = 0; q < kPlanWords; ++q) plan_w[q] = src[q];
  }
  // (the partial block's loads stay ahead of the row's, so that waiting for
  // them leaves those in flight)
  __builtin_amdgcn_sched_barrier(0);
  const int wbase = (w >> 1) * kNpBlock + (w & 1) * (kNpBlock / 2) + 4 * lane;
  float v[64];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const float4 e = MODE == 2 ? *reinterpret_cast<const float4*>(xr + wbase + 256 * k)
                               : ld_stream4(xr + wbase + 256 * k);
    v[4 * k] = e.x;
    v[4 * k + 1] = e.y;
    v[4 * k + 2] = e.z;
    v[4 * k + 3] = e.w;
  }
#pragma unroll
  for (int i = 0; i < TPT; ++i) {
    const int e = 4 * (t + i * NT);
    if (e < m) *reinterpret_cast<float4*>(res_tail + np_pad(e)) = u[i];
  }
  __syncthreads();

  // numpy's sums of f over the partial block's leaves, eight lanes a leaf,
  // into tv (LDS only)
  auto tail_leaves = [&](auto f) {
    const int j = t & 7;
    for (int leaf = t >> 3; leaf < nleaf; leaf += NT / 8) {  // uniform over the leaf's lanes
      const int lo = p_lo[leaf], n = p_n[leaf];
      float res = 0.0f;
      if (n < 8) {
        if (j == 0)
          for (int i = 0; i < n; ++i) res += f(res_tail[np_pad(lo + i)]);
      } else {
        // the accumulator's terms (at most sixteen) read together, indexes
        // held inside the partial block, the ones past the body left out
        const int body = n - n % 8;
        float term[kNpLeaf / 8];
#pragma unroll
        for (int k = 0; k < kNpLeaf / 8; ++k)
          term[k] = f(res_tail[np_pad(min(lo + 8 * k + j, m - 1))]);
        float q = term[0];
#pragma unroll
        for (int k = 1; k < kNpLeaf / 8; ++k)
          if (8 * k < body) q += term[k];
        q += dpp_move<0xB1, 0xF>(q, 0.0f);   // lane pairs (xor 1)
        q += dpp_move<0x4E, 0xF>(q, 0.0f);   // quads (xor 2)
        q += dpp_move<0x141, 0xF>(q, 0.0f);  // eights (row half mirror: xor 4 once quads agree)
        res = q;
        if (j == 0)
          for (int i = body; i < n; ++i) res += f(res_tail[np_pad(lo + i)]);
      }
      if (j == 0) tv[leaf] = res;
    }
  };
  // wave 0, after tail_leaves and a barrier: the partial block's tree, a
  // level at a time (LDS accesses of one wave take effect in order); its root
  auto tail_tree = [&]() -> float {
    if (!nleaf) return 0.0f;
    for (int l = 0; l < A.tail.nlev; ++l) {
      const int k = (l ? A.tail.lev_end[l - 1] : 0) + lane;
      if (k < A.tail.lev_end[l]) tv[nleaf + k] = tv[p_ca[k]] + tv[p_cb[k]];
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
    return tv[A.tail.nnode ? nleaf + A.tail.nnode - 1 : 0];
  };
  float* const stg = res_lds + A.stage_off + w * 8 * kPitch;
  // Chunk Q (leaves 8Q .. 8Q+7 of the wave, v[16Q .. 16Q+15] in load
  // order) turned in place, through the wave's stage, into numpy's order:
  // lane 8 q + j then holds the sixteen terms of accumulator j of leaf q.
  auto to_leaf_order = [&](auto Qc) {
    constexpr int Q = decltype(Qc)::value;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int pos = 256 * r + 4 * lane;
      *reinterpret_cast<float4*>(stg + (pos >> 7) * kPitch + (pos & 127)) =
          make_float4(v[16 * Q + 4 * r], v[16 * Q + 4 * r + 1], v[16 * Q + 4 * r + 2],
                      v[16 * Q + 4 * r + 3]);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    const float* src = stg + (lane >> 3) * kPitch + (lane & 7);
#pragma unroll
    for (int k = 0; k < 16; ++k) v[16 * Q + k] = src[8 * k];
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
  };
  // the wave's 32 leaves of f, from registers; lane 0 leaves their balanced
  // sum in ws[w]
  auto wave_leaves = [&](auto f) {
    float part[4];
#pragma unroll
    for (int Q = 0; Q < 4; ++Q) {
      float a = f(v[16 * Q]);
#pragma unroll
      for (int k = 1; k < 16; ++k) a += f(v[16 * Q + k]);
      // lane pairs, quads, eights (the leaf's eight accumulators), then
      // leaf pairs, fours and eights: each DPP stage adds the same two
      // partial sums as an xor butterfly over 1, 2, 4, 8, 16, 32, so the
      // total (lane 63's) carries the balanced tree's roundings
      part[Q] = wave_sum_dpp(a);
    }
    if (lane == 0) ws[w] = (part[0] + part[1]) + (part[2] + part[3]);  // the wave's 32 leaves
  };
  // wave 0, after a barrier: numpy's loop over the 8192-blocks, acc = 0,
  // acc += each whole block, then the partial block's sum
  auto block_loop = [&](float tail_sum) -> float {
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < NB; ++b) acc += ws[2 * b] + ws[2 * b + 1];
    if (nleaf) acc += tail_sum;
    return acc;
  };

  // the sum of x: the partial block's leaves and tree first, while the row's
  // loads are still arriving
  auto ident = [](float e) { return e; };
  tail_leaves(ident);
  __syncthreads();
  const float ts1 = w == 0 ? tail_tree() : 0.0f;
  to_leaf_order(std::integral_constant<int, 0>{});
  to_leaf_order(std::integral_constant<int, 1>{});
  to_leaf_order(std::integral_constant<int, 2>{});
  to_leaf_order(std::integral_constant<int, 3>{});
  wave_leaves(ident);
  __syncthreads();
  if (w == 0 && lane == 0) bc[0] = block_loop(ts1);
  __syncthreads();
  const float n = static_cast<float>(A.T);
  const float mean = bc[0] / n;
  // the sum of (x - mean)^2 (tv and ws free again: wave 0 read them before
  // the last barrier)
  auto sqdev = [mean](float e) {
    const float d = e - mean;
    return d * d;
  };
  wave_leaves(sqdev);
  tail_leaves(sqdev);
  __syncthreads();
  if (w == 0) {
    const float ts2 = tail_tree();
    if (lane == 0) bc[1] = block_loop(ts2);
  }
  __syncthreads();
  const float den = sqrtf(bc[1] / n + A.eps);
  const int64_t c = row % A.C;
  float gamma = 0.0f, beta = 0.0f;
  if (A.af.mode == 1) { gamma = A.af.gb[c]; beta = A.af.gb[A.C + c]; }
  const RowAffine ra = row_affine(A.af, A.C, c, gamma, beta);
  const KkDivisor dv = kk_divisor(den);
  if constexpr (MODE == 0) {
    float* orow = A.out + row * A.T;
    auto y4 = [&](float4 e) {
      const float4 q = kk_div4(make_float4(e.x - mean, e.y - mean, e.z - mean, e.w - mean), dv);
      return make_float4(apply_affine<false>(q.x, ra, A.af), apply_affine<false>(q.y, ra, A.af),
                         apply_affine<false>(q.z, ra, A.af), apply_affine<false>(q.w, ra, A.af));
    };
    // y in leaf order, then back to load order through the stage, chunk by
    // chunk, for 1 KB stores
#pragma unroll
    for (int Q = 0; Q < 4; ++Q) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 y = y4(make_float4(v[16 * Q + 4 * g], v[16 * Q + 4 * g + 1],
                                        v[16 * Q + 4 * g + 2], v[16 * Q + 4 * g + 3]));
        float* dst = stg + (lane >> 3) * kPitch + (lane & 7) + 32 * g;
        dst[0] = y.x;
        dst[8] = y.y;
        dst[16] = y.z;
        dst[24] = y.w;
      }
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int pos = 256 * r + 4 * lane;
        st_stream4(orow + wbase + 256 * (4 * Q + r),
                   *reinterpret_cast<const float4*>(stg + (pos >> 7) * kPitch + (pos & 127)));
      }
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
    float* ot = orow + NB * kNpBlock;
    for (int e = 4 * t; e < m; e += 4 * NT)
      st_stream4(ot + e, y4(*reinterpret_cast<const float4*>(res_tail + np_pad(e))));
  } else {
    // the row's x extremes; y is monotonic in x up to rounding (the caller
    // checks every y against the bounds where it may not be)
    float lo = v[0], hi = v[0];
#pragma unroll
    for (int k = 1; k < 64; ++k) {
      lo = fminf(lo, v[k]);
      hi = fmaxf(hi, v[k]);
    }
    for (int e = 4 * t; e < m; e += 4 * NT) {
      const float4 x4 = *reinterpret_cast<const float4*>(res_tail + np_pad(e));
      lo = fminf(fminf(lo, x4.x), fminf(fminf(x4.y, x4.z), x4.w));
      hi = fmaxf(fmaxf(hi, x4.x), fmaxf(fmaxf(x4.y, x4.z), x4.w));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      lo = fminf(lo, __shfl_xor(lo, off, 64));
      hi = fmaxf(hi, __shfl_xor(hi, off, 64));
    }
    if (lane == 0) wmm[w] = make_float2(lo, hi);
    __syncthreads();
    if (w == 0) {
      lo = wmm[0].x;
      hi = wmm[0].y;
      for (int i = 1; i < NT / 64; ++i) {
        lo = fminf(lo, wmm[i].x);
        hi = fmaxf(hi, wmm[i].y);
      }
      // even lanes at xmin, odd at xmax
      const float y = apply_affine(kk_div(((lane & 1) ? hi : lo) - mean, dv), ra, A.af);
      const float y1 = __shfl_xor(y, 1, 64);
      if (lane == 0) {
        A.stats[row] = make_float2(mean, den);
        A.mm[row] = make_float2(fminf(y, y1), fmaxf(y, y1));
      }
    }
  }
}

// Rows of at most 128 elements (one numpy leaf), one thread per row.
__global__ void np_leaf_rows_kernel(float* __restrict__ out, const float* __restrict__ x,
                                    int64_t rows, int n, int mean) {
  const int64_t row = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (row >= rows) return;
  const float* a = x + row * n;
  float res = 0.0f;
  if (n < 8) {
    for (int i = 0; i < n; ++i) res += a[i];
  } else {
    float r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = a[j];
    const int body = n - n % 8;
    for (int i = 8; i < body; i += 8)
#pragma unroll
      for (int j = 0; j < 8; ++j) r[j] += a[i + j];
    res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (int i = body; i < n; ++i) res += a[i];
  }
  res = 0.0f + res;  // the reduction's accumulator starts at 0
  out[row] = mean ? res / static_cast<float>(n) : res;
}

// General reduction: kept axes (kdims/kst) index the output in order,
// reduced axes (rdims/rst) are walked by each thread; x is strided.
struct RedArgs {
  int kr, rr;
  int64_t kdims[KK_MAX_RANK], kst[KK_MAX_RANK];
  int64_t rdims[KK_MAX_RANK], rst[KK_MAX_RANK];
  int64_t nout, nred;
};

__global__ void reduce_generic_kernel(float* __restrict__ out, const float* __restrict__ x,
                                      RedArgs R, int op) {
  for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < R.nout;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t rem = t, base = 0;
    for (int d = R.kr - 1; d >= 0; --d) {
      base += (rem % R.kdims[d]) * R.kst[d];
      rem /= R.kdims[d];
    }
    float s = 0.0f;  // numpy sums a non-contiguous axis in order, in fp32
    float m = -INFINITY;
    bool nan = false;
    if (R.rr == 1) {
      // One reduced axis: sixteen independent loads in flight, then added
      // (or compared) in order.
      const int64_t st = R.rst[0];
      int64_t j = 0;
      for (; j + 16 <= R.nred; j += 16) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = x[base + (j + u) * st];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          s += v[u];
          nan |= __builtin_isnan(v[u]);
          m = fmaxf(m, v[u]);
        }
      }
      for (; j < R.nred; ++j) {
        const float v = x[base + j * st];
        s += v;
        nan |= __builtin_isnan(v);
        m = fmaxf(m, v);
      }
    }
    for (int64_t j = 0; j < R.nred && R.rr != 1; ++j) {
      int64_t rj = j, off = base;
      for (int d = R.rr - 1; d >= 0; --d) {
        off += (rj % R.rdims[d]) * R.rst[d];
        rj /= R.rdims[d];
      }
      const float v = x[off];
      s += v;
      nan |= __builtin_isnan(v);
      m = fmaxf(m, v);
    }
    float v;
    if (op == KK_REDUCE_MAX) v = nan ? NAN : m;
    else if (op == KK_REDUCE_MEAN) v = s / static_cast<float>(R.nred);
    else v = s;
    out[t] = v;
  }
}

// ------------------------------------------------------------- launching
// Picks (GROUP, NV, VEC) so that GROUP * NV * VEC covers the row; returns
// false when the row is too long for registers.
struct RowShape {
  int group, nv, vec;
};
static bool pick_row_shape(int64_t n, bool vec_ok, RowShape* rs) {
  const int vec = vec_ok ? 4 : 1;
  const int64_t nvec = ceil_div(n, vec);
  static const int nvs[] = {1, 2, 4, 8, 16};
  // One wavefront per row while the row fits 64 * 4 vectors (keeps many
  // rows in flight for short rows); 256 threads per row beyond that.
  for (int nv : nvs) {
    if (nv > 4) break;
    if (nvec <= int64_t(64) * nv) { *rs = {64, nv, vec}; return true; }
  }
  for (int nv : nvs)
    if (nvec <= int64_t(256) * nv) { *rs = {256, nv, vec}; return true; }
  return false;
}

// One-wave rows go four to a 256-thread block, or one to a 64-thread block
// when four to a block would leave fewer than two blocks per CU.
static unsigned row_threads(const RowShape& rs, int64_t rows) {
  const int64_t cus = ctx().num_cus > 0 ? ctx().num_cus : 256;
  return rs.group == 64 && ceil_div(rows, kRowBlock / 64) < 2 * cus ? 64u : unsigned(kRowBlock);
}

#define KK_ROW_DISPATCH(KERNEL, RS, GRID_ROWS, ...)                                          \
  do {                                                                                         \
    const unsigned _threads = row_threads((RS), (GRID_ROWS));                                  \
    const int _rpb = static_cast<int>(_threads) / (RS).group;                                  \
    const dim3 _grid(static_cast<unsigned>(ceil_div((GRID_ROWS), _rpb)));                      \
    hipStream_t _s = ctx().stream;                                                             \
    if ((RS).group == 64) {                                                                    \
      if ((RS).vec == 4) {                                                                     \
        switch ((RS).nv) {                                                                     \
          case 1: KK_LAUNCH((KERNEL<64, 1, 4>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
          case 2: KK_LAUNCH((KERNEL<64, 2, 4>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
          default: KK_LAUNCH((KERNEL<64, 4, 4>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
        }                                                                                      \
      } else {                                                                                 \
        switch ((RS).nv) {                                                                     \
          case 1: KK_LAUNCH((KERNEL<64, 1, 1>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
          case 2: KK_LAUNCH((KERNEL<64, 2, 1>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
          default: KK_LAUNCH((KERNEL<64, 4, 1>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
        }                                                                                      \
      }                                                                                        \
    } else {                                                                                   \
      if ((RS).vec == 4) {                                                                     \
        switch ((RS).nv) {                                                                     \
          case 1: KK_LAUNCH((KERNEL<256, 1, 4>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
          case 2: KK_LAUNCH((KERNEL<256, 2, 4>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
          case 4: KK_LAUNCH((KERNEL<256, 4, 4>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
          case 8: KK_LAUNCH((KERNEL<256, 8, 4>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
          default: KK_LAUNCH((KERNEL<256, 16, 4>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
        }                                                                                      \
      } else {                                                                                 \
        switch ((RS).nv) {                                                                     \
          case 1: KK_LAUNCH((KERNEL<256, 1, 1>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
          case 2: KK_LAUNCH((KERNEL<256, 2, 1>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
          case 4: KK_LAUNCH((KERNEL<256, 4, 1>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
          case 8: KK_LAUNCH((KERNEL<256, 8, 1>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
          default: KK_LAUNCH((KERNEL<256, 16, 1>), _grid, dim3(_threads), 0, _s, __VA_ARGS__); break; \
        }                                                                                      \
      }                                                                                        \
    }                                                                                          \
  } while (0)

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

static int check_f32_contig(const kk_tensor* t, const char* name) {
  KK_TRY(check_tensor(t, name));
  if (t->dtype != KK_F32) return set_error(KK_E_ARG, "%s must be fp32", name);
  if (!is_contiguous(t)) return set_error(KK_E_ARG, "%s must be contiguous", name);
  return KK_OK;
}

static bool same_shape(const kk_tensor* a, const kk_tensor* b) {
  if (a->rank != b->rank) return false;
  for (int i = 0; i < a->rank; ++i)
    if (a->shape[i] != b->shape[i]) return false;
  return true;
}

constexpr int64_t kNpRowMax = 15000;  // rows held in LDS (<= 64 KB with padding)

// Spacing of the per-row counters: up to 32 ints (128 bytes) apart.
static int counter_stride(int64_t rows) {
  int st = 32;
  while (st > 1 && rows * st > kRowCounters) st >>= 1;
  return st;
}

static size_t np_row_lds(int64_t n) {
  return sizeof(float) * static_cast<size_t>(n + 8 * ceil_div(n, kNpLeaf));
}

// numpy's pairwise tree over the m elements of a row's partial last block
// (0 <= m < 8192) as an NpTail: the leaves as np_leaves lists them, the
// internal nodes ordered by height.
static void np_tail_plan(int m, NpTail* P) {
  *P = NpTail{};
  P->m = m;
  if (m <= 0) return;
  struct Node {
    int a, b, h;  // children: id >= 0 a leaf, else internal node -1 - id
  };
  std::vector<Node> nodes;
  auto rec = [&](auto&& self, int lo, int n) -> std::pair<int, int> {  // (id, height)
    if (n <= kNpLeaf) {
      P->lo[P->nleaf] = static_cast<uint16_t>(lo);
      P->n[P->nleaf] = static_cast<uint8_t>(n);
      return {P->nleaf++, 0};
    }
    int n2 = n / 2;
    n2 -= n2 % 8;
    const auto l = self(self, lo, n2);
    const auto r = self(self, lo + n2, n - n2);
    nodes.push_back({l.first, r.first, 1 + std::max(l.second, r.second)});
    return {-static_cast<int>(nodes.size()), nodes.back().h};
  };
  rec(rec, 0, m);
  std::vector<int> order(nodes.size()), pos(nodes.size());
  std::iota(order.begin(), order.end(), 0);
  std::stable_sort(order.begin(), order.end(),
                   [&](int a, int b) { return nodes[a].h < nodes[b].h; });
  for (size_t i = 0; i < order.size(); ++i) pos[order[i]] = static_cast<int>(i);
  auto id = [&](int c) { return static_cast<uint8_t>(c >= 0 ? c : P->nleaf + pos[-1 - c]); };
  P->nnode = static_cast<int>(nodes.size());
  for (size_t i = 0; i < order.size(); ++i) {
    const Node& nd = nodes[order[i]];
    P->ca[i] = id(nd.a);
    P->cb[i] = id(nd.b);
    P->nlev = std::max(P->nlev, nd.h);
    P->lev_end[nd.h - 1] = static_cast<uint8_t>(i + 1);
  }
}

// Sum / mean of rows of x (rows x n, contiguous) in numpy's order.
static int np_reduce_rows(float* out, const float* x, int64_t rows, int64_t n, bool mean,
                          bool vec) {
  hipStream_t st = ctx().stream;
  NpTail tail;  // the rows' partial 8192-block, if any
  np_tail_plan(static_cast<int>(n % kNpBlock), &tail);
  if (n <= kNpLeaf) {
    KK_LAUNCH(np_leaf_rows_kernel, dim3(static_cast<unsigned>(ceil_div(rows, 256))),
                       dim3(256), 0, st, out, x, rows, static_cast<int>(n), mean ? 1 : 0);
    return check_launch("np_leaf_rows_kernel");
  }
  if (n <= kNpRowMax) {
    Affine af{};
    KK_LAUNCH(np_rows_kernel, dim3(static_cast<unsigned>(rows)), dim3(kNpThreads),
                       np_row_lds(n), st, out, x, int64_t{1}, static_cast<int>(n), mean ? 1 : 0,
                       0.0f, af, vec ? 1 : 0, static_cast<float2*>(nullptr), static_cast<float2*>(nullptr),
                       tail);
    return check_launch("np_rows_kernel");
  }
  if (rows > kRowCounters) return set_error(KK_E_UNSUPPORTED, "reduce: %lld long rows", (long long)rows);
  const int64_t nblk = ceil_div(n, kNpBlock);
  void* part = nullptr;
  KK_TRY(kk_alloc(sizeof(float) * rows * nblk, &part));
  KK_LAUNCH(np_blocks_kernel, dim3(static_cast<unsigned>(nblk), static_cast<unsigned>(rows)),
                     dim3(kNpThreads), 0, st, static_cast<float*>(part), x, n,
                     static_cast<int>(nblk), 0, static_cast<float2*>(nullptr), ctx().row_counters,
                     counter_stride(rows), out, mean ? 1 : 0, 0.0f, static_cast<float2*>(nullptr),
                     static_cast<float2*>(nullptr), int64_t{0}, Affine{}, tail,
                     static_cast<const float*>(nullptr), int64_t{0});
  const int rc = check_launch("np_blocks_kernel");
  kk_free(part);  // stream order keeps it alive for the kernel
  return rc;
}

// Rows np_resident_kernel takes: 15000 < T < 9 * 8192 (one to eight whole
// 8192-blocks and a partial one), T % 4 == 0, x 16-byte aligned.
static bool np_resident_ok(int64_t T, const void* x) {
  return T > kNpRowMax && T < 9 * kNpBlock && T % 4 == 0 && aligned16(x);
}

// out set: writes y (MODE 0; no snake); else stats and mm (MODE 2).
static int np_resident_launch(float* out, const float* x, int64_t rows, int64_t C, int64_t T,
                              float eps, const Affine& af, float2* stats, float2* mm) {
  ResArgs A{};
  A.out = out;
  A.x = x;
  A.stats = stats;
  A.mm = mm;
  A.C = C;
  A.T = T;
  A.eps = eps;
  A.af = af;
  // the delayed half (rows of one wave of blocks, at most one a CU; with
  // more rows than CUs later blocks start staggered anyway): the other
  // half's bytes at 6.1 TB/s (what one block a row reads at when no block
  // stores), in ticks of the 100 MHz clock (s_memrealtime)
  const int64_t cus = ctx().num_cus > 0 ? ctx().num_cus : 256;
  if (out && 4 * rows >= 3 * cus && rows <= cus)
    A.delay = static_cast<int>(0.5 * static_cast<double>(rows * T) * 4.0 / 6.1e12 * 1e8);

  const int nb = static_cast<int>(T / kNpBlock);
  np_tail_plan(static_cast<int>(T - nb * kNpBlock), &A.tail);
  // the partial block, then 8 leaves of 136 floats a wave
  A.stage_off = static_cast<int>(ceil_div(static_cast<int64_t>(np_row_lds(A.tail.m)), 16) * 4);
  const size_t lds = 4 * static_cast<size_t>(A.stage_off) +
                     sizeof(float) * (2 * nb) * 8 * (kNpLeaf + 8);
  const dim3 grid(static_cast<unsigned>(rows));
  hipStream_t st = ctx().stream;
#define KK_RES_CASE(NBV)                                                                          \
  case NBV:                                                                                       \
    if (out) KK_LAUNCH((np_resident_kernel<NBV, 0>), grid, dim3(128 * NBV), lds, st, A); \
    else KK_LAUNCH((np_resident_kernel<NBV, 2>), grid, dim3(128 * NBV), lds, st, A);  \
    break;
  switch (nb) {
    KK_RES_CASE(1)
    KK_RES_CASE(2)
    KK_RES_CASE(3)
    KK_RES_CASE(4)
    KK_RES_CASE(5)
    KK_RES_CASE(6)
    KK_RES_CASE(7)
    KK_RES_CASE(8)
    default:
      return set_error(KK_E_UNSUPPORTED, "instance norm: no resident kernel for T = %lld", (long long)T);
  }
#undef KK_RES_CASE
  return check_launch("np_resident_kernel");
}

// Instance norm with the statistics in numpy's order (modes 0, 1, 3).
static int instnorm_np(const kk_tensor* out, const kk_tensor* x, int64_t rows, int64_t C,
                       int64_t T, float eps, const Affine& af, bool vec_ok) {
  hipStream_t st = ctx().stream;
  NpTail tail;  // the rows' partial 8192-block, if any
  np_tail_plan(static_cast<int>(T % kNpBlock), &tail);
  const float* xp = static_cast<const float*>(x->data);
  if (T <= kNpRowMax) {
    KK_LAUNCH(np_rows_kernel, dim3(static_cast<unsigned>(rows)), dim3(kNpThreads),
                       np_row_lds(T), st, static_cast<float*>(out->data), xp, C,
                       static_cast<int>(T), 2, eps, af, vec_ok ? 1 : 0, static_cast<float2*>(nullptr),
                       static_cast<float2*>(nullptr), tail);
    return check_launch("np_rows_kernel");
  }
  if (np_resident_ok(T, x->data) && aligned16(out->data) && !af.snake_a)
    return np_resident_launch(static_cast<float*>(out->data), xp, rows, C, T, eps, af, nullptr,
                              nullptr);
  if (rows > kRowCounters)
    return set_error(KK_E_UNSUPPORTED, "instance norm: %lld long rows", (long long)rows);
  const int64_t nblk = ceil_div(T, kNpBlock);
  const int64_t part_bytes = ceil_div(static_cast<int64_t>(sizeof(float)) * rows * nblk, 256) * 256;
  void* ws = nullptr;
  KK_TRY(kk_alloc(static_cast<size_t>(part_bytes + sizeof(float2) * rows), &ws));
  float* part = static_cast<float*>(ws);
  float2* stats = reinterpret_cast<float2*>(static_cast<char*>(ws) + part_bytes);
  // pass 0: the sums, then the mean; pass 1: the squared deviations' sums,
  // then sqrt(var + eps); then the normalisation
  const dim3 bgrid(static_cast<unsigned>(nblk), static_cast<unsigned>(rows));
  int rc = KK_OK;
  for (int pass = 0; pass < 2 && rc == KK_OK; ++pass) {
    KK_LAUNCH(np_blocks_kernel, bgrid, dim3(kNpThreads), 0, st, part, xp, T,
                       static_cast<int>(nblk), pass, stats, ctx().row_counters,
                       counter_stride(rows), static_cast<float*>(nullptr), 0, eps,
                       static_cast<float2*>(nullptr), static_cast<float2*>(nullptr), int64_t{0},
                       Affine{}, tail, static_cast<const float*>(nullptr), int64_t{0});
    rc = check_launch("np_blocks_kernel");
  }
  if (rc == KK_OK) {
    // any row length vectorises once both bases are 16-byte aligned
    const bool avec = aligned16(x->data) && aligned16(out->data);
    const int64_t per_block = kRowBlock * (avec ? 4 : 1) * 8;
    const unsigned gx = static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(
        ceil_div(T, per_block), 1 << 16)));
    KK_LAUNCH(instnorm_apply, dim3(gx, static_cast<unsigned>(rows)), dim3(kRowBlock), 0,
                       st, static_cast<float*>(out->data), xp, static_cast<const float2*>(stats), C,
                       T, af, avec ? 1 : 0);
    rc = check_launch("instnorm_apply");
  }
  kk_free(ws);  // stream order keeps it alive for the kernels above
  return rc;
}

// The instance norm chain (with its affine, LeakyRelu or snake) and the
// DynamicQuantizeLinear that alone reads its result, without storing the
// float result y.  Rows held in LDS: one pass for the statistics and the
// rows' (min, max) of y, then one that recomputes y and writes its bytes.
// Long rows: the two statistics passes, the first also taking each row's
// (min, max) of x; y is monotonic in x per row (the affine, a LeakyRelu
// with alpha >= 0, and the snake y + sin^2(a y) / a, whose slope is
// 1 + sin(2 a y) >= 0), so y at those two points bounds the row and the
// extremes over all rows give the quantiser's scale and zero point.  Where
// rounding could break that (the snake: sin's last bit), the quantising pass
// checks every y against the bounds and, if one falls outside, flags it,
// and each of its blocks leaves the exact (min, max) of its y; two more
// launches that do nothing unless flagged then fold those partials into
// the scale and zero point again and write the bytes again.
// A value per InstanceNormQuant call for its out-of-bounds flag, never 0
// (wraps after 2^31 - 1 calls).
static int next_epoch() {
  static uint32_t n = 0;
  n = n % 0x7ffffffeu + 1u;
  return static_cast<int>(n);
}

static int instnorm_quant_run(const kk_tensor* q, const kk_tensor* y_scale, const kk_tensor* y_zp,
                              const kk_tensor* x, float eps, const Affine& af,
                              const float* leaves = nullptr) {
  hipStream_t st = ctx().stream;
  const int64_t T = x->shape[x->rank - 1];
  const int64_t C = x->shape[x->rank - 2];
  const int64_t rows = numel(x) / T;
  NpTail tail;  // the rows' partial 8192-block, if any
  np_tail_plan(static_cast<int>(T % kNpBlock), &tail);
  const float* xp = static_cast<const float*>(x->data);
  // the quantising pass vectorises any row length once the bases are
  // aligned; the rows held in LDS take 16-byte loads only when T % 4 == 0
  const bool vec = aligned16(x->data) && (reinterpret_cast<uintptr_t>(q->data) % 4 == 0);
  const bool rows_vec = vec && T % 4 == 0;
  const int64_t per_block = kRowBlock * (vec ? 4 : 1) * 8;
  const int64_t gx = std::max<int64_t>(1, std::min<int64_t>(ceil_div(T, per_block), 1 << 16));
  const bool long_rows = T > kNpRowMax;
  if (long_rows && rows > kRowCounters)
    return set_error(KK_E_UNSUPPORTED, "instance norm: %lld long rows", (long long)rows);
  // y is monotonic in x with exact floats: no snake, and a LeakyRelu slope >= 0
  const bool exact_bounds = !af.snake_a && (!af.leaky || af.alpha >= 0.0f);
  const int64_t nblk = long_rows ? ceil_div(T, kNpBlock) : 0;
  // the quantising pass's per-block (min, max) of y, kept for the fallback
  const int64_t nbmm = long_rows && !exact_bounds ? rows * gx : 0;
  if (nbmm > 0x7fffffff) return set_error(KK_E_UNSUPPORTED, "instance norm: too many partials");
  auto up = [](int64_t b) { return ceil_div(b, 256) * 256; };
  const int64_t o_stats = 0, o_mm = up(8 * rows), o_par = o_mm + up(8 * rows);
  const int64_t o_part = o_par + 256, o_xmm = o_part + up(4 * rows * nblk + 4);
  const int64_t o_flag = o_xmm + up(8 * rows * nblk + 8), o_bmm = o_flag + 256;
  const int64_t total = o_bmm + up(8 * nbmm);
  void* ws = nullptr;
  KK_TRY(kk_alloc(static_cast<size_t>(total), &ws));
  char* base = static_cast<char*>(ws);
  float2* stats = reinterpret_cast<float2*>(base + o_stats);
  float2* mm = reinterpret_cast<float2*>(base + o_mm);
  float2* params = reinterpret_cast<float2*>(base + o_par);
  float* part = reinterpret_cast<float*>(base + o_part);
  float2* xmm = reinterpret_cast<float2*>(base + o_xmm);
  int* flag = long_rows && !exact_bounds ? reinterpret_cast<int*>(base + o_flag) : nullptr;
  float2* bmm = flag ? reinterpret_cast<float2*>(base + o_bmm) : nullptr;
  float* ysp = static_cast<float*>(y_scale->data);
  uint8_t* yzp = static_cast<uint8_t*>(y_zp->data);
  const dim3 qgrid(static_cast<unsigned>(gx), static_cast<unsigned>(rows));
  // the fallback quantising launch (rarely flagged) takes about 2048
  // blocks, so that an unflagged one ends at once; its loops stride over
  // the rows
  const int64_t fgx = std::min<int64_t>(gx, std::max<int64_t>(1, ceil_div(2048, rows)));
  const dim3 fgrid(static_cast<unsigned>(fgx), static_cast<unsigned>(rows));
  // Up to 2048 rows every quantising block folds the rows' (min, max)
  // partials itself; beyond, a dql_fold launch folds them into params.
  const bool fold_in = rows <= 2048;
  const int epoch = next_epoch();
  auto quant = [&](const int* only_if, int* check, const float2* fold, int64_t npart) {
    KK_LAUNCH(instnorm_quant, only_if ? fgrid : qgrid, dim3(kRowBlock), 0, st,
                       static_cast<uint8_t*>(q->data), xp, static_cast<const float2*>(stats),
                       static_cast<const float2*>(params), fold, static_cast<int>(npart), ysp,
                       yzp, C, T, af, vec ? 1 : 0, only_if, check, epoch, check ? bmm : nullptr);
    return check_launch("instnorm_quant");
  };
  int rc = KK_OK;
  if (!long_rows) {
    KK_LAUNCH(np_rows_kernel, dim3(static_cast<unsigned>(rows)), dim3(kNpThreads),
                       np_row_lds(T), st, static_cast<float*>(nullptr), xp, C, static_cast<int>(T), 3,
                       eps, af, rows_vec ? 1 : 0, stats, mm, tail);
    rc = check_launch("np_rows_kernel");
  } else if (np_resident_ok(T, x->data)) {
    rc = np_resident_launch(nullptr, xp, rows, C, T, eps, af, stats, mm);
  } else {
    const dim3 bgrid(static_cast<unsigned>(nblk), static_cast<unsigned>(rows));
    for (int pass = 0; pass < 2 && rc == KK_OK; ++pass) {
      KK_LAUNCH(np_blocks_kernel, bgrid, dim3(kNpThreads), 0, st, part, xp, T,
                         static_cast<int>(nblk), pass, stats, ctx().row_counters,
                         counter_stride(rows), static_cast<float*>(nullptr), 0, eps, xmm,
                         pass == 1 ? mm : static_cast<float2*>(nullptr), C, af, tail, leaves,
                         (T / kNpBlock) * 64);
      rc = check_launch("np_blocks_kernel");
    }
  }
  // (dql_fold with clear zeroes the flag; folded in, the flag is compared
  // with this call's epoch instead)
  if (rc == KK_OK && !fold_in)
    rc = launch_dql_fold(mm, static_cast<int>(rows), params, ysp, yzp, nullptr, flag);
  if (rc == KK_OK) rc = quant(nullptr, flag, fold_in ? mm : nullptr, rows);
  if (rc == KK_OK && flag) {  // only if a y fell outside the bounds: the
    // exact (min, max) from that pass's block partials, and the bytes again;
    // up to 16384 partials (the 128-id graph's [1,128,405840]: 6400) every
    // block of the second quantising pass folds them itself, so an
    // unflagged call adds one launch that ends at once, not two
    if (nbmm <= 16384) {
      rc = quant(flag, nullptr, bmm, nbmm);
    } else {
      rc = launch_dql_fold(bmm, static_cast<int>(nbmm), params, ysp, yzp, flag, nullptr, epoch);
      if (rc == KK_OK) rc = quant(flag, nullptr, nullptr, rows);
    }
  }
  kk_free(ws);  // stream order keeps it alive for the kernels above
  return rc;
}

static int instnorm_launch(const kk_tensor* out, const kk_tensor* x, float eps, const Affine& af,
                           const StyleArgs& sa) {
  if (x->rank < 2) return set_error(KK_E_ARG, "instance norm: x must be [N, C, ...T]");
  const int64_t T = x->shape[x->rank - 1];
  const int64_t C = x->shape[x->rank - 2];
  const int64_t rows = numel(x) / (T ? T : 1);
  if (numel(x) == 0) return KK_OK;
  RowShape rs;
  const bool vec_ok = (T % 4 == 0) && aligned16(x->data) && aligned16(out->data);
  if (af.mode != 2) return instnorm_np(out, x, rows, C, T, eps, af, vec_ok);
  const int64_t nvec = T / 4;
  if (vec_ok && nvec > 4 * kRowBlock && nvec <= 16 * kRowBlock) {
    const int nv = static_cast<int>(ceil_div(nvec, 512));
    const dim3 grid(static_cast<unsigned>(rows));
    const float it = 1.0f / static_cast<float>(T);
    float* op = static_cast<float*>(out->data);
    const float* xp = static_cast<const float*>(x->data);
    hipStream_t st = ctx().stream;
    switch (nv) {
      case 3: KK_LAUNCH((instnorm_wide_kernel<8, 3>), grid, dim3(512), 0, st, op, xp, C, T, it, eps, sa); break;
      case 4: KK_LAUNCH((instnorm_wide_kernel<8, 4>), grid, dim3(512), 0, st, op, xp, C, T, it, eps, sa); break;
      case 5: KK_LAUNCH((instnorm_wide_kernel<8, 5>), grid, dim3(512), 0, st, op, xp, C, T, it, eps, sa); break;
      case 6: KK_LAUNCH((instnorm_wide_kernel<8, 6>), grid, dim3(512), 0, st, op, xp, C, T, it, eps, sa); break;
      default: KK_LAUNCH((instnorm_wide_kernel<8, 8>), grid, dim3(512), 0, st, op, xp, C, T, it, eps, sa); break;
    }
    return check_launch("instnorm_wide_kernel");
  }
  if (vec_ok && nvec > 4 * 64 && nvec <= 8 * 64) {
    // One wave per row (T up to 2048, the decoder's [1,512,1200]): its sums
    // are DPP moves within the wave, with no LDS round or barrier, and each
    // lane keeps its 5-8 vectors' loads in flight together.
    const int nv = static_cast<int>(ceil_div(nvec, 64));
    const dim3 grid(static_cast<unsigned>(rows));
    float* op = static_cast<float*>(out->data);
    const float* xp = static_cast<const float*>(x->data);
    hipStream_t st = ctx().stream;
    const int Ti = static_cast<int>(T);  // (T <= 2048 here)
    const float it = 1.0f / static_cast<float>(T);
    switch (nv) {
      case 5: KK_LAUNCH((adain_row_kernel<5>), grid, dim3(64), 0, st, op, xp, C, Ti, it, eps, sa); break;
      case 6: KK_LAUNCH((adain_row_kernel<6>), grid, dim3(64), 0, st, op, xp, C, Ti, it, eps, sa); break;
      case 7: KK_LAUNCH((adain_row_kernel<7>), grid, dim3(64), 0, st, op, xp, C, Ti, it, eps, sa); break;
      default: KK_LAUNCH((adain_row_kernel<8>), grid, dim3(64), 0, st, op, xp, C, Ti, it, eps, sa); break;
    }
    return check_launch("adain_row_kernel");
  }
  if (pick_row_shape(T, vec_ok, &rs)) {
    KK_ROW_DISPATCH(instnorm_kernel, rs, rows, static_cast<float*>(out->data),
                    static_cast<const float*>(x->data), rows, C, T, eps, af, sa);
  } else {
    KK_LAUNCH(instnorm_long_kernel, dim3(static_cast<unsigned>(rows)), dim3(kRowBlock), 0,
                       ctx().stream, static_cast<float*>(out->data),
                       static_cast<const float*>(x->data), C, T, eps, af, sa);
  }
  return check_launch("instnorm_kernel");
}

// A per-channel operand of x [N, C, T]: C values that broadcast along T, i.e.
// shaped [..., C, 1] (or any shape of one value when C is 1).  A [C] operand
// would broadcast along T instead, so it is not one.
static bool per_channel(const kk_tensor* t, const kk_tensor* x, int64_t C) {
  if (numel(t) != C || t->rank > x->rank) return false;
  if (C == 1) return true;
  return t->rank >= 2 && t->shape[t->rank - 1] == 1 && t->shape[t->rank - 2] == C;
}

static int instance_norm_scale_shift(const kk_tensor* out, const kk_tensor* x,
                                     const kk_tensor* scale, const kk_tensor* shift,
                                     const kk_tensor* snake_a, const kk_tensor* snake_r, float eps,
                                     int leaky, float alpha, const kk_tensor* y_scale = nullptr,
                                     const kk_tensor* y_zp = nullptr,
                                     const kk_tensor* leaves = nullptr) {
  KK_TRY(require_ready());
  KK_TRY(check_f32_contig(x, "x"));
  KK_TRY(check_tensor(out, "out"));
  if (y_scale) {  // out is the quantised result
    KK_TRY(check_tensor(y_scale, "y_scale"));
    KK_TRY(check_tensor(y_zp, "y_zero_point"));
    if (out->dtype != KK_U8 || !is_contiguous(out) || y_scale->dtype != KK_F32 ||
        numel(y_scale) != 1 || y_zp->dtype != KK_U8 || numel(y_zp) != 1)
      return set_error(KK_E_ARG, "instance norm quant: y uint8 like x, scale one fp32, zero point "
                                 "one uint8");
  } else {
    KK_TRY(check_f32_contig(out, "out"));
  }
  if (out->rank != x->rank || numel(out) != numel(x))
    return set_error(KK_E_ARG, "instance norm: out shape must equal x");
  for (int i = 0; i < x->rank; ++i)
    if (out->shape[i] != x->shape[i]) return set_error(KK_E_ARG, "instance norm: out shape must equal x");
  if (x->rank < 2) return set_error(KK_E_ARG, "instance norm: x must be [N, C, ...T]");
  const int64_t C = x->shape[x->rank - 2];
  Affine af{};
  af.mode = 3;
  af.leaky = leaky ? 1 : 0;
  af.alpha = alpha;
  for (const kk_tensor* t : {scale, shift}) {
    if (!t) continue;
    KK_TRY(check_f32_contig(t, t == scale ? "scale" : "shift"));
    if (!per_channel(t, x, C))
      return set_error(KK_E_ARG, "instance norm: scale/shift need C = %lld values shaped "
                       "[..., C, 1]", (long long)C);
  }
  af.scale = scale ? static_cast<const float*>(scale->data) : nullptr;
  af.shift = shift ? static_cast<const float*>(shift->data) : nullptr;
  if (snake_a) {
    for (const kk_tensor* t : {snake_a, snake_r}) {
      KK_TRY(check_f32_contig(t, t == snake_a ? "snake alpha" : "snake recip"));
      if (!per_channel(t, x, C))
        return set_error(KK_E_ARG, "instance norm: snake alpha/recip need C = %lld values shaped "
                         "[..., C, 1]",
                         (long long)C);
    }
    af.snake_a = static_cast<const float*>(snake_a->data);
    af.snake_r = static_cast<const float*>(snake_r->data);
  }
  if (y_scale) {
    if (numel(x) == 0) return set_error(KK_E_ARG, "instance norm quant: empty input");
    const float* lv = nullptr;
    if (leaves) {
      const int64_t T = x->shape[x->rank - 1], rows = numel(x) / T;
      if (!leaf_matches(leaves->data, x->data, rows, T))
        return set_error(KK_E_ARG, "kk_instance_norm_quant_leaves: leaves were not formed from x");
      lv = static_cast<const float*>(leaves->data);
    }
    return instnorm_quant_run(out, y_scale, y_zp, x, eps, af, lv);
  }
  StyleArgs sa{};
  return instnorm_launch(out, x, eps, af, sa);
}

}  // namespace kk

using namespace kk;

extern "C" {

int kk_instance_norm_affine(const kk_tensor* out, const kk_tensor* x, const kk_tensor* gamma_beta,
                            float eps) {
  KK_TRY(require_ready());
  KK_TRY(check_f32_contig(x, "x"));
  KK_TRY(check_f32_contig(out, "out"));
  if (!same_shape(out, x)) return set_error(KK_E_ARG, "instance norm: out shape must equal x");
  const float* gb = nullptr;
  if (gamma_beta) {
    KK_TRY(check_f32_contig(gamma_beta, "gamma_beta"));
    const int64_t C = x->rank >= 2 ? x->shape[x->rank - 2] : 0;
    if (numel(gamma_beta) != 2 * C)
      return set_error(KK_E_ARG, "instance norm: gamma_beta needs 2C = %lld elements",
                       (long long)(2 * C));
    gb = static_cast<const float*>(gamma_beta->data);
  }
  StyleArgs sa{};
  Affine af{};
  af.mode = gb ? 1 : 0;
  af.gb = gb;
  return instnorm_launch(out, x, eps, af, sa);
}

int kk_instance_norm_scale_shift(const kk_tensor* out, const kk_tensor* x, const kk_tensor* scale,
                                 const kk_tensor* shift, float eps, int leaky, float alpha) {
  return instance_norm_scale_shift(out, x, scale, shift, nullptr, nullptr, eps, leaky, alpha);
}

int kk_instance_norm_quant(const kk_tensor* y, const kk_tensor* y_scale, const kk_tensor* y_zp,
                           const kk_tensor* x, const kk_tensor* scale, const kk_tensor* shift,
                           const kk_tensor* alpha, const kk_tensor* recip, float eps, int leaky,
                           float leaky_alpha) {
  if ((alpha == nullptr) != (recip == nullptr))
    return set_error(KK_E_ARG, "kk_instance_norm_quant: snake needs both alpha and recip");
  if (alpha && leaky)
    return set_error(KK_E_UNSUPPORTED, "kk_instance_norm_quant: LeakyRelu and snake together");
  if (!y_scale || !y_zp) return set_error(KK_E_ARG, "kk_instance_norm_quant: scale/zero point outputs");
  return instance_norm_scale_shift(y, x, scale, shift, alpha, recip, eps, leaky, leaky_alpha,
                                   y_scale, y_zp);
}

int kk_instance_norm_quant_leaves(const kk_tensor* y, const kk_tensor* y_scale,
                                  const kk_tensor* y_zp, const kk_tensor* x,
                                  const kk_tensor* scale, const kk_tensor* shift,
                                  const kk_tensor* alpha, const kk_tensor* recip, float eps,
                                  int leaky, float leaky_alpha, const kk_tensor* leaves) {
  if ((alpha == nullptr) != (recip == nullptr))
    return set_error(KK_E_ARG, "kk_instance_norm_quant_leaves: snake needs both alpha and recip");
  if (alpha && leaky)
    return set_error(KK_E_UNSUPPORTED, "kk_instance_norm_quant_leaves: LeakyRelu and snake together");
  if (!y_scale || !y_zp)
    return set_error(KK_E_ARG, "kk_instance_norm_quant_leaves: scale/zero point outputs");
  return instance_norm_scale_shift(y, x, scale, shift, alpha, recip, eps, leaky, leaky_alpha,
                                   y_scale, y_zp, leaves);
}

int kk_instance_norm_scale_shift_snake(const kk_tensor* out, const kk_tensor* x,
                                       const kk_tensor* scale, const kk_tensor* shift,
                                       const kk_tensor* alpha, const kk_tensor* recip, float eps) {
  if (!alpha || !recip)
    return set_error(KK_E_ARG, "kk_instance_norm_scale_shift_snake: alpha and recip are required");
  return instance_norm_scale_shift(out, x, scale, shift, alpha, recip, eps, 0, 0.0f);
}

int kk_adain(const kk_tensor* out, const kk_tensor* x, const kk_tensor* style, const kk_tensor* w,
             const kk_tensor* w_scale, const kk_tensor* w_zp, const kk_tensor* bias, float eps) {
  KK_TRY(require_ready());
  KK_TRY(check_f32_contig(x, "x"));
  KK_TRY(check_f32_contig(out, "out"));
  KK_TRY(check_f32_contig(style, "style"));
  KK_TRY(check_tensor(w, "w"));
  if (!same_shape(out, x)) return set_error(KK_E_ARG, "adain: out shape must equal x");
  if (x->rank < 2) return set_error(KK_E_ARG, "adain: x must be [N, C, T]");
  const int64_t C = x->shape[x->rank - 2];
  const int64_t S = numel(style);
  if (w->rank != 2 || w->shape[0] != S || w->shape[1] != 2 * C)
    return set_error(KK_E_ARG, "adain: w must be [S=%lld, 2C=%lld]", (long long)S,
                     (long long)(2 * C));
  if (x->shape[0] != 1 && x->rank == 3)
    return set_error(KK_E_UNSUPPORTED, "adain: one style row serves batch 1 only");
  StyleArgs sa{};
  sa.style = static_cast<const float*>(style->data);
  sa.w = w->data;
  sa.w_dt = w->dtype;
  sa.w_sk = w->strides[0];
  sa.w_sj = w->strides[1];
  sa.S = S;
  KK_TRY(make_dequant(&sa.dq, w, w_scale, w_zp, 2 * C, "adain"));
  if (bias) {
    KK_TRY(check_f32_contig(bias, "bias"));
    if (numel(bias) != 2 * C) return set_error(KK_E_ARG, "adain: bias needs 2C elements");
    sa.bias = static_cast<const float*>(bias->data);
  }
  Affine af{};
  af.mode = 2;
  return instnorm_launch(out, x, eps, af, sa);
}

int kk_layernorm(const kk_tensor* out, const kk_tensor* x, const kk_tensor* skip,
                 const kk_tensor* skip_bias, const kk_tensor* scale, const kk_tensor* bias,
                 int axis, float eps) {
  KK_TRY(require_ready());
  KK_TRY(check_f32_contig(x, "x"));
  KK_TRY(check_f32_contig(out, "out"));
  KK_TRY(check_f32_contig(scale, "scale"));
  if (!same_shape(out, x)) return set_error(KK_E_ARG, "layernorm: out shape must equal x");
  if (axis < 0) axis += x->rank;
  if (axis < 0 || axis >= x->rank) return set_error(KK_E_ARG, "layernorm: axis out of range");
  int64_t cols = 1;
  for (int i = axis; i < x->rank; ++i) cols *= x->shape[i];
  const int64_t n = numel(x);
  if (n == 0) return KK_OK;
  const int64_t rows = n / cols;
  if (numel(scale) != cols) return set_error(KK_E_ARG, "layernorm: scale needs %lld elements", (long long)cols);
  LnArgs la{};
  la.scale = static_cast<const float*>(scale->data);
  if (bias) {
    KK_TRY(check_f32_contig(bias, "bias"));
    if (numel(bias) != cols) return set_error(KK_E_ARG, "layernorm: bias needs %lld elements", (long long)cols);
    la.bias = static_cast<const float*>(bias->data);
  }
  if (skip) {
    KK_TRY(check_f32_contig(skip, "skip"));
    if (!same_shape(skip, x)) return set_error(KK_E_ARG, "layernorm: skip shape must equal x");
    la.skip = static_cast<const float*>(skip->data);
    if (skip_bias) {
      KK_TRY(check_f32_contig(skip_bias, "skip_bias"));
      if (numel(skip_bias) != cols) return set_error(KK_E_ARG, "layernorm: skip bias needs %lld elements", (long long)cols);
      la.skip_bias = static_cast<const float*>(skip_bias->data);
    }
  } else if (skip_bias) {
    return set_error(KK_E_ARG, "layernorm: skip_bias without skip");
  }
  bool vec_ok = (cols % 4 == 0) && aligned16(x->data) && aligned16(out->data) &&
                aligned16(la.scale) && (!la.bias || aligned16(la.bias)) &&
                (!la.skip || aligned16(la.skip)) && (!la.skip_bias || aligned16(la.skip_bias));
  const int64_t nvec = cols / 4;
  if (vec_ok && !la.skip && nvec > 64 && nvec <= 8 * 64) {
    const int nv = static_cast<int>(ceil_div(nvec, 64));
    const dim3 grid(static_cast<unsigned>(rows));
    float* op = static_cast<float*>(out->data);
    const float* xp = static_cast<const float*>(x->data);
    const int ci = static_cast<int>(cols);
    const float ic = 1.0f / static_cast<float>(cols);
    hipStream_t st = ctx().stream;
#define KK_LN_ROW(NVV)                                                                        \
  if (la.bias)                                                                                \
    KK_LAUNCH((layernorm_row_kernel<NVV, true>), grid, dim3(64), 0, st, op, xp, ci,  \
                       ic, eps, la.scale, la.bias);                                           \
  else                                                                                        \
    KK_LAUNCH((layernorm_row_kernel<NVV, false>), grid, dim3(64), 0, st, op, xp, ci, \
                       ic, eps, la.scale, la.bias);
    switch (nv) {
      case 2: KK_LN_ROW(2) break;
      case 3: KK_LN_ROW(3) break;
      case 4: KK_LN_ROW(4) break;
      case 5: KK_LN_ROW(5) break;
      case 6: KK_LN_ROW(6) break;
      case 7: KK_LN_ROW(7) break;
      default: KK_LN_ROW(8) break;
    }
#undef KK_LN_ROW
    return check_launch("layernorm_row_kernel");
  }
  RowShape rs;
  if (pick_row_shape(cols, vec_ok, &rs)) {
    KK_ROW_DISPATCH(layernorm_kernel, rs, rows, static_cast<float*>(out->data),
                    static_cast<const float*>(x->data), rows, cols, eps, la);
  } else {
    KK_LAUNCH(layernorm_long_kernel, dim3(static_cast<unsigned>(rows)), dim3(kRowBlock), 0,
                       ctx().stream, static_cast<float*>(out->data),
                       static_cast<const float*>(x->data), cols, eps, la);
  }
  return check_launch("layernorm_kernel");
}

int kk_softmax(const kk_tensor* out, const kk_tensor* x, int axis) {
  KK_TRY(require_ready());
  KK_TRY(check_f32_contig(x, "x"));
  KK_TRY(check_f32_contig(out, "out"));
  if (!same_shape(out, x)) return set_error(KK_E_ARG, "softmax: out shape must equal x");
  if (x->rank == 0) return set_error(KK_E_ARG, "softmax: scalar input");
  if (axis < 0) axis += x->rank;
  if (axis < 0 || axis >= x->rank) return set_error(KK_E_ARG, "softmax: axis out of range");
  int64_t outer = 1, inner = 1;
  for (int i = 0; i < axis; ++i) outer *= x->shape[i];
  for (int i = axis + 1; i < x->rank; ++i) inner *= x->shape[i];
  const int64_t dim = x->shape[axis];
  if (numel(x) == 0) return KK_OK;
  RowShape rs;
  const bool vec_ok = (dim % 4 == 0) && aligned16(x->data) && aligned16(out->data);
  if (inner == 1 && pick_row_shape(dim, vec_ok, &rs)) {
    KK_ROW_DISPATCH(softmax_kernel, rs, outer, static_cast<float*>(out->data),
                    static_cast<const float*>(x->data), outer, dim);
    return check_launch("softmax_kernel");
  }
  const int64_t cols = outer * inner;
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>(ceil_div(cols, 256), 65535));
  KK_LAUNCH(softmax_cols_kernel, dim3(grid), dim3(256), 0, ctx().stream,
                     static_cast<float*>(out->data), static_cast<const float*>(x->data), outer, dim,
                     inner);
  return check_launch("softmax_cols_kernel");
}

int kk_reduce(int op, const kk_tensor* out, const kk_tensor* x, uint32_t axes_mask) {
  KK_TRY(require_ready());
  KK_TRY(check_tensor(x, "x"));
  KK_TRY(check_f32_contig(out, "out"));
  if (x->dtype != KK_F32) return set_error(KK_E_ARG, "reduce: x must be fp32");
  if (op != KK_REDUCE_SUM && op != KK_REDUCE_MEAN && op != KK_REDUCE_MAX)
    return set_error(KK_E_ARG, "reduce: unknown op %d", op);
  if (axes_mask >> x->rank) return set_error(KK_E_ARG, "reduce: axis beyond rank");
  RedArgs R{};
  int64_t nout = 1, nred = 1;
  for (int i = 0; i < x->rank; ++i) {
    if (axes_mask & (1u << i)) {
      R.rdims[R.rr] = x->shape[i];
      R.rst[R.rr++] = x->strides[i];
      nred *= x->shape[i];
    } else {
      R.kdims[R.kr] = x->shape[i];
      R.kst[R.kr++] = x->strides[i];
      nout *= x->shape[i];
    }
  }
  if (numel(out) != nout) return set_error(KK_E_ARG, "reduce: out has %lld elements, expected %lld",
                                           (long long)numel(out), (long long)nout);
  R.nout = nout;
  R.nred = nred;
  if (nout == 0) return KK_OK;
  if (nred == 0) {
    // numpy: sum of nothing is 0, mean of nothing is NaN, max raises.
    if (op == KK_REDUCE_MAX) return set_error(KK_E_ARG, "reduce: max over an empty axis");
    return kk_fill(out, op == KK_REDUCE_SUM ? 0.0 : NAN);
  }
  // Fast path: contiguous x whose reduced axes are exactly the trailing ones.
  bool trailing = is_contiguous(x);
  {
    bool seen_red = false;
    for (int i = 0; i < x->rank && trailing; ++i) {
      const bool red = axes_mask & (1u << i);
      if (red) seen_red = true;
      else if (seen_red && x->shape[i] != 1) trailing = false;
    }
  }
  RowShape rs;
  const bool vec_ok = (nred % 4 == 0) && aligned16(x->data);
  if (trailing && op != KK_REDUCE_MAX)
    return np_reduce_rows(static_cast<float*>(out->data), static_cast<const float*>(x->data), nout,
                          nred, op == KK_REDUCE_MEAN, vec_ok);
  if (trailing && pick_row_shape(nred, vec_ok, &rs)) {
    KK_ROW_DISPATCH(reduce_rows_kernel, rs, nout, static_cast<float*>(out->data),
                    static_cast<const float*>(x->data), nout, nred, op);
    return check_launch("reduce_rows_kernel");
  }
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>(ceil_div(nout, 256), 65535));
  KK_LAUNCH(reduce_generic_kernel, dim3(grid), dim3(256), 0, ctx().stream,
                     static_cast<float*>(out->data), static_cast<const float*>(x->data), R, op);
  return check_launch("reduce_generic_kernel");
}

}  // extern "C"
