// The waveform's output stage, as runtime/audio.gd:59-106 drives it: the
// notch FIR (kernels/fir.glsl:35-47) and the float -> 16-bit PCM conversion
// (kernels/pcm16.glsl:28-46), separately or fused into one pass.
//
// FIR: y[i] = sum_k h[k] x[clamp(i - center + k, 0, n - 1)], each output's
// taps accumulated in order (k = 0, 1, ...) in fp32 with one fused
// multiply-add per tap.  A block of 256 threads computes 2048 consecutive
// outputs: it stages the input window they read (2048 + taps - 1 samples,
// edges clamped) in LDS once; each thread keeps a 16-sample register window
// over its 8 consecutive outputs and slides it 8 taps at a time (two 16-byte
// LDS reads per 64 FMAs), the taps coming from the scalar cache (the same
// address in every lane).  1023 taps over 2.15M samples are 2.2 G FMAs:
// bound by the VALU's fp32 FMA rate, not by HBM (17 MB in and out).
//
// PCM16: round(clamp(x * gain, -1, 1) * 32767) as int16, written as the
// little-endian byte stream the reference reads back (two bytes per
// sample).  GLSL's round() leaves a .5 tie to the implementation; roundf
// rounds it away from zero.
#include <algorithm>
#include <type_traits>

#include "kk_internal.h"

namespace kk {
namespace audio {  // named: the kernels keep readable names in profiles

constexpr int kThreads = 256;
constexpr int kPerThread = 8;                        // consecutive outputs per thread
constexpr int kTile = kThreads * kPerThread;         // outputs per block
constexpr int kMaxTaps = 4096;                       // window: kTile + taps rounded up + slack
constexpr int kWindow = kTile + kMaxTaps + 16;

__device__ __forceinline__ int16_t to_pcm16(float v, float gain) {
  const float c = fminf(fmaxf(v * gain, -1.0f), 1.0f);
  return static_cast<int16_t>(roundf(c * 32767.0f));
}

// PCM: pcm16 bytes out instead of fp32 (the fused form).
template <bool PCM>
__global__ void __launch_bounds__(kThreads) fir_kernel(const float* __restrict__ x, int64_t n,
                                                       const float* __restrict__ h, int taps,
                                                       int center, float* __restrict__ y,
                                                       int16_t* __restrict__ pcm, float gain) {
  __shared__ __align__(16) float xs[kWindow];
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * kTile;
  const int taps8 = (taps + 7) & ~7;
  const int span = kTile + taps8 + 8;  // the window the threads read
  for (int j = threadIdx.x; j < span; j += kThreads) {
    int64_t s = i0 - center + j;
    s = s < 0 ? 0 : (s >= n ? n - 1 : s);
    xs[j] = x[s];
  }
  __syncthreads();
  const int j0 = threadIdx.x * kPerThread;
  float acc[kPerThread];
#pragma unroll
  for (int r = 0; r < kPerThread; ++r) acc[r] = 0.0f;
  float win[16];
  {
    const float4 a = *reinterpret_cast<const float4*>(&xs[j0]);
    const float4 b = *reinterpret_cast<const float4*>(&xs[j0 + 4]);
    win[0] = a.x; win[1] = a.y; win[2] = a.z; win[3] = a.w;
    win[4] = b.x; win[5] = b.y; win[6] = b.z; win[7] = b.w;
  }
  // eight taps: slide the window by 8 and accumulate (the taps are the same
  // address in every lane: scalar loads); `tail` guards a partial last chunk
  auto chunk = [&](int k0, auto tail) {
    const float4 a = *reinterpret_cast<const float4*>(&xs[j0 + k0 + 8]);
    const float4 b = *reinterpret_cast<const float4*>(&xs[j0 + k0 + 12]);
    win[8] = a.x; win[9] = a.y; win[10] = a.z; win[11] = a.w;
    win[12] = b.x; win[13] = b.y; win[14] = b.z; win[15] = b.w;
    float hk[8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      hk[kk] = (!decltype(tail)::value || k0 + kk < taps) ? h[k0 + kk] : 0.0f;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
#pragma unroll
      for (int r = 0; r < kPerThread; ++r) acc[r] = __builtin_fmaf(hk[kk], win[r + kk], acc[r]);
#pragma unroll
    for (int q = 0; q < 8; ++q) win[q] = win[q + 8];
  };
  const int full = taps & ~7;
  for (int k0 = 0; k0 < full; k0 += 8) chunk(k0, std::false_type{});
  if (full < taps) chunk(full, std::true_type{});
  const int64_t o = i0 + j0;
  if (o + kPerThread <= n) {
    if (PCM) {
      uint32_t w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        w[q] = static_cast<uint16_t>(to_pcm16(acc[2 * q], gain)) |
               (static_cast<uint32_t>(static_cast<uint16_t>(to_pcm16(acc[2 * q + 1], gain))) << 16);
      *reinterpret_cast<uint4*>(pcm + o) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
      st_stream4(y + o, make_float4(acc[0], acc[1], acc[2], acc[3]));
      st_stream4(y + o + 4, make_float4(acc[4], acc[5], acc[6], acc[7]));
    }
  } else {
#pragma unroll
    for (int r = 0; r < kPerThread; ++r) {
      if (o + r >= n) break;
      if (PCM) pcm[o + r] = to_pcm16(acc[r], gain);
      else y[o + r] = acc[r];
    }
  }
}

// Eight samples per thread: two 16-byte loads, one 16-byte store.
__global__ void __launch_bounds__(256) pcm16_kernel(const float* __restrict__ x, int64_t n,
                                                    float gain, int16_t* __restrict__ pcm) {
  const int64_t n8 = n / 8;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n8; i += stride) {
    const float4 a = ld_stream4(x + 8 * i);
    const float4 b = ld_stream4(x + 8 * i + 4);
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      w[q] = static_cast<uint16_t>(to_pcm16(v[2 * q], gain)) |
             (static_cast<uint32_t>(static_cast<uint16_t>(to_pcm16(v[2 * q + 1], gain))) << 16);
    *reinterpret_cast<uint4*>(pcm + 8 * i) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  // the last n % 8 samples, one per thread of the grid's first threads
  const int64_t t = 8 * n8 + blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (t < n) pcm[t] = to_pcm16(x[t], gain);
}

}  // namespace audio
using namespace audio;

// x: contiguous fp32 waveform (any shape); out_bytes: contiguous uint8 with
// 2 * numel(x) elements.
static int check_wave(const kk_tensor* x, const char* who) {
  KK_TRY(require_ready());
  KK_TRY(check_tensor(x, "x"));
  if (x->dtype != KK_F32 || !is_contiguous(x))
    return set_error(KK_E_ARG, "%s: x must be a contiguous fp32 waveform", who);
  if (reinterpret_cast<uintptr_t>(x->data) % 16)
    return set_error(KK_E_ARG, "%s: x must be 16-byte aligned", who);
  return KK_OK;
}

static int check_pcm_out(const kk_tensor* out, int64_t n, const char* who) {
  KK_TRY(check_tensor(out, "out"));
  if (out->dtype != KK_U8 || !is_contiguous(out) || numel(out) != 2 * n)
    return set_error(KK_E_ARG, "%s: out must be contiguous uint8 with 2 * %lld bytes", who,
                     (long long)n);
  if (reinterpret_cast<uintptr_t>(out->data) % 16)
    return set_error(KK_E_ARG, "%s: out must be 16-byte aligned", who);
  return KK_OK;
}

static int check_taps(const kk_tensor* taps, int* center, const char* who) {
  KK_TRY(check_tensor(taps, "taps"));
  const int64_t t = numel(taps);
  if (taps->dtype != KK_F32 || !is_contiguous(taps) || t < 1 || t > kMaxTaps)
    return set_error(KK_E_ARG, "%s: taps must be contiguous fp32 with 1..%d values", who, kMaxTaps);
  if (*center < 0) *center = static_cast<int>((t - 1) / 2);
  if (*center >= t) return set_error(KK_E_ARG, "%s: center %d outside the %lld taps", who, *center,
                                     (long long)t);
  return KK_OK;
}

static int launch_fir(const kk_tensor* x, const kk_tensor* taps, int center, float* y, int16_t* pcm,
                      float gain) {
  const int64_t n = numel(x);
  const int64_t blocks = ceil_div(n, kTile);
  if (blocks > 0x7fffffff) return set_error(KK_E_UNSUPPORTED, "FIR: waveform too long");
  const float* xp = static_cast<const float*>(x->data);
  const float* hp = static_cast<const float*>(taps->data);
  const int t = static_cast<int>(numel(taps));
  if (pcm)
    KK_LAUNCH(fir_kernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                       ctx().stream, xp, n, hp, t, center, nullptr, pcm, gain);
  else
    KK_LAUNCH(fir_kernel<false>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                       ctx().stream, xp, n, hp, t, center, y, nullptr, 0.0f);
  return check_launch("fir_kernel");
}

}  // namespace kk

using namespace kk;

extern "C" {

int kk_fir(const kk_tensor* out, const kk_tensor* x, const kk_tensor* taps, int center) {
  KK_TRY(check_wave(x, "kk_fir"));
  KK_TRY(check_taps(taps, &center, "kk_fir"));
  KK_TRY(check_tensor(out, "out"));
  if (out->dtype != KK_F32 || !is_contiguous(out) || numel(out) != numel(x) ||
      reinterpret_cast<uintptr_t>(out->data) % 16)
    return set_error(KK_E_ARG, "kk_fir: out must be a 16-byte-aligned contiguous fp32 tensor of x's size");
  if (numel(x) == 0) return KK_OK;
  return launch_fir(x, taps, center, static_cast<float*>(out->data), nullptr, 0.0f);
}

int kk_pcm16(const kk_tensor* out_bytes, const kk_tensor* x, float gain) {
  KK_TRY(check_wave(x, "kk_pcm16"));
  const int64_t n = numel(x);
  KK_TRY(check_pcm_out(out_bytes, n, "kk_pcm16"));
  if (n == 0) return KK_OK;
  const unsigned g = static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 8 * 256), 4096)));
  KK_LAUNCH(pcm16_kernel, dim3(g), dim3(256), 0, ctx().stream,
                     static_cast<const float*>(x->data), n, gain, static_cast<int16_t*>(out_bytes->data));
  return check_launch("pcm16_kernel");
}

int kk_fir_pcm16(const kk_tensor* out_bytes, const kk_tensor* x, const kk_tensor* taps, int center,
                 float gain) {
  KK_TRY(check_wave(x, "kk_fir_pcm16"));
  KK_TRY(check_taps(taps, &center, "kk_fir_pcm16"));
  const int64_t n = numel(x);
  KK_TRY(check_pcm_out(out_bytes, n, "kk_fir_pcm16"));
  if (n == 0) return KK_OK;
  return launch_fir(x, taps, center, nullptr, static_cast<int16_t*>(out_bytes->data), gain);
}

}  // extern "C"
