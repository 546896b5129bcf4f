// ConvInteger on the int8 matrix cores (v_mfma_i32_32x32x32_i8), exact in
// int32 (op_conv_integer, ref_runtime.py:130-134: conv of (x - x_zp) with
// (w - w_zp), padding contributing 0 after the shift).
//
// Both uint8 operands are offset into int8 (u - 128), so a product of
// shifted values expands as
//   sum_k (a_k - wz')(b_k - xz') = sum_k a_k b_k - xz' sum_k a_k
//                                  - wz' sum_k b_k + K wz' xz'
// with a = w - 128 (uint8 weights; int8 weights are used as they are),
// b = x - 128, wz' and xz' the zero points offset the same way.  Padded time
// positions hold b = xz', so they contribute 0 exactly as the reference's
// zero padding of the shifted input does.
//
// Layout: the weights become wT[Cout][Kw][CinP] and the activations
// xT[N][Lp][CinP] (time-major, channels contiguous, CinP = Cin rounded up
// to 64 with zero channels), so each MFMA operand fragment -- 16 channels
// of one tap at one output row or time step -- is one 16-byte load.  The
// prep kernels also produce sum_k a_k per output channel and
// sum_ci b[t][ci] per time step for the epilogue.
#include "kk_internal.h"

namespace kk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kTileM = 128;  // output channels per block (2 waves x 64)
constexpr int kCinAlign = 64;   // channels per chunk: two 32-deep MFMA steps
constexpr int kRowPitch = 80;   // LDS bytes per 64-channel row (16-byte pad: staggered banks)

// wT[co][tap][ci] = offset weight (0 for padding rows/channels);
// wsum[co] = sum of the offset weights; wzo[co] = offset weight zero point.
__global__ void __launch_bounds__(256) conv_i8_wprep(const void* __restrict__ w, int w_dt,
                                                     const void* __restrict__ wzp, int wzp_dt,
                                                     int64_t wzp_n, int8_t* __restrict__ wT,
                                                     int32_t* __restrict__ wsum,
                                                     int32_t* __restrict__ wzo, int64_t Cout,
                                                     int64_t Cin, int64_t Kw, int64_t CinP) {
  __shared__ int part[4];
  const int64_t co = blockIdx.x;
  const bool live = co < Cout;
  const int off = w_dt == KK_U8 ? 128 : 0;
  int local = 0;
  for (int64_t idx = threadIdx.x; idx < Kw * CinP; idx += blockDim.x) {
    const int64_t tap = idx / CinP, ci = idx % CinP;
    int a = 0;
    if (live && ci < Cin) {
      const int64_t src = (co * Cin + ci) * Kw + tap;
      a = w_dt == KK_U8 ? static_cast<int>(static_cast<const uint8_t*>(w)[src]) - 128
                        : static_cast<int>(static_cast<const int8_t*>(w)[src]);
    }
    wT[(co * Kw + tap) * CinP + ci] = static_cast<int8_t>(a);
    local += a;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) local += __shfl_xor(local, o, 64);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) part[wv] = local;
  __syncthreads();
  if (threadIdx.x == 0) {
    wsum[co] = live ? part[0] + part[1] + part[2] + part[3] : 0;
    int z = 0;  // padding rows: a = 0, so any value works; keep 0
    if (live) z = (wzp ? static_cast<int>(load_as_i64(wzp, wzp_dt, wzp_n > 1 ? co : 0)) : 0) - off;
    wzo[co] = z;
  }
}

// xT[b][t][ci] = x[b][ci][t - p0] - 128 for t inside the signal, xz - 128 in
// the padding, 0 in the padding channels; xs[b][t] = sum over real channels.
// A block owns 64 time steps and walks the channels in tiles of 64: lane l
// of wave w loads x[ci][t0 + l] for ci = w, w + 4, ... (64 consecutive bytes
// per load), the tile is transposed through LDS, and each thread stores 16
// consecutive channels of one time step as one 16-byte store.
constexpr int kPrepT = 64;   // time steps per block
constexpr int kPrepC = 64;   // channels per tile

__global__ void __launch_bounds__(256) conv_i8_xprep(const uint8_t* __restrict__ x,
                                                     const uint8_t* __restrict__ xzp,
                                                     int8_t* __restrict__ xT,
                                                     int32_t* __restrict__ xs, int64_t Cin,
                                                     int64_t L, int64_t p0, int64_t Lp,
                                                     int64_t CinP) {
  __shared__ int8_t tile[kPrepC][kPrepT + 4];
  __shared__ int part[4][kPrepT];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kPrepT;
  const int64_t b = blockIdx.y;
  const int pad = (xzp ? static_cast<int>(xzp[0]) : 0) - 128;
  const uint8_t* xb = x + b * Cin * L;
  // loader: time step t0 + lane
  const int64_t ts = t0 + lane - p0;
  const bool inside = ts >= 0 && ts < L;
  // storer: time step t0 + lane, channels 16 * wv .. 16 * wv + 15 of the tile
  const int64_t to = t0 + lane;
  int sum = 0;
  for (int64_t c0 = 0; c0 < CinP; c0 += kPrepC) {
#pragma unroll
    for (int k = 0; k < kPrepC / 4; ++k) {
      const int r = wv + 4 * k;
      const int64_t ci = c0 + r;
      int v = 0;
      if (ci < Cin) v = inside ? static_cast<int>(xb[ci * L + ts]) - 128 : pad;
      tile[r][lane] = static_cast<int8_t>(v);
    }
    __syncthreads();
    if (to < Lp && c0 + 16 * wv < CinP) {
      v4i pack;
      int8_t* pv = reinterpret_cast<int8_t*>(&pack);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        pv[e] = tile[16 * wv + e][lane];
        sum += pv[e];
      }
      *reinterpret_cast<v4i*>(xT + (b * Lp + to) * CinP + c0 + 16 * wv) = pack;
    }
    __syncthreads();
  }
  part[wv][lane] = sum;
  __syncthreads();
  if (wv == 0 && to < Lp) xs[b * Lp + to] = (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]);
}

struct ConvI8Args {
  const int8_t* wT;     // [CoutP][Kw][CinP]
  const int32_t* wsum;  // [CoutP]
  const int32_t* wzo;   // [CoutP]
  const int8_t* xT;     // [N][Lp][CinP]
  const int32_t* xs;    // [N][Lp]
  const uint8_t* xzp;   // one uint8 or NULL
  int32_t* out;         // [N][Cout][Lout] int32, or NULL when outf is set
  float* outf;          // [N][Cout][Lout] float(acc + bias[co]) * scale
  const int32_t* bias;  // [Cout] or NULL
  const float* scale;   // 1 or Cout values
  int64_t scale_n;
  int64_t Cout, CinP, Kw, s, d, Lp, Lout, Kreal;
  int W;                // time rows of a block's input window
};

// Block: 128 output channels x TN output steps, 4 waves as 2 (channels) x
// 2 (time), wave tile 64 x TN/2 as 2 x TN/64 MFMA tiles of 32 x 32.  For each
// 64-channel chunk the block stages its whole input window -- the
// ((TN - 1) s + (K - 1) d + 1) time rows every tap reads, each tap shifted by
// tap * d -- in LDS once, and streams the 128 x 64 weight tile of each tap
// through a double buffer (the next tap's tile is fetched into registers
// while this tap's MFMAs run).  Lane (r, g) = (lane % 32, lane / 32) reads
// A[r][16g .. 16g+15] and B[16g .. 16g+15][r] of each 32 x 32 x 32 step
// from LDS; D(i, j) lands in lane j + 32 ((i / 4) % 2), register
// (i / 8) 4 + i % 4.
// TN (128 or 64) output steps per block; a wave covers TN / 2 of them.
template <int TN>
__global__ void __launch_bounds__(256) conv_i8_kernel(ConvI8Args A) {
  constexpr int NI = TN / 64;  // 32-wide MFMA tiles per wave along time
  extern __shared__ __align__(16) int8_t conv_lds[];
  int8_t* Bw = conv_lds;                             // [W][kRowPitch]
  int8_t* As = conv_lds + A.W * kRowPitch;           // [2][kTileM][kRowPitch]
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int r = lane & 31, g = lane >> 5;
  const int wm = wv >> 1, wn = wv & 1;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kTileM;
  const int64_t nb = static_cast<int64_t>(blockIdx.x) * TN;
  const int64_t b = blockIdx.z;
  const int8_t* xT = A.xT + b * A.Lp * A.CinP;
  const int64_t tw0 = nb * A.s;
  // weight-tile loader: 128 rows x four 16-byte pieces, two per thread
  auto load_a = [&](int64_t tap, int64_t c0, v4i (&reg)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int q = tid + 256 * j, row = q >> 2, c = q & 3;
      reg[j] = *reinterpret_cast<const v4i*>(A.wT + ((m0 + row) * A.Kw + tap) * A.CinP + c0 +
                                              16 * c);
    }
  };
  auto store_a = [&](int buf, const v4i (&reg)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int q = tid + 256 * j, row = q >> 2, c = q & 3;
      *reinterpret_cast<v4i*>(As + (buf * kTileM + row) * kRowPitch + 16 * c) = reg[j];
    }
  };
  v16i acc[2][NI] = {};
  for (int64_t c0 = 0; c0 < A.CinP; c0 += kCinAlign) {
    // The input window; rows past the signal's end are clamped in bounds
    // (their outputs are never stored).
    for (int q = tid; q < A.W * 4; q += 256) {
      const int row = q >> 2, c = q & 3;
      int64_t t = tw0 + row;
      t = t < A.Lp ? t : A.Lp - 1;
      *reinterpret_cast<v4i*>(Bw + row * kRowPitch + 16 * c) =
          *reinterpret_cast<const v4i*>(xT + t * A.CinP + c0 + 16 * c);
    }
    v4i ra[2];
    load_a(0, c0, ra);
    store_a(0, ra);
    __syncthreads();
    for (int64_t tap = 0; tap < A.Kw; ++tap) {
      const int buf = static_cast<int>(tap & 1);
      if (tap + 1 < A.Kw) load_a(tap + 1, c0, ra);
      const int8_t* Ab = As + buf * kTileM * kRowPitch;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int col = ks * 32 + 16 * g;
        v4i af[2], bf[NI];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
          af[mi] = *reinterpret_cast<const v4i*>(Ab + (wm * 64 + mi * 32 + r) * kRowPitch + col);
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
          const int64_t row = (wn * (TN / 2) + ni * 32 + r) * A.s + tap * A.d;
          bf[ni] = *reinterpret_cast<const v4i*>(Bw + row * kRowPitch + col);
        }
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
          for (int ni = 0; ni < NI; ++ni)
            acc[mi][ni] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[mi], bf[ni], acc[mi][ni], 0, 0, 0);
      }
      if (tap + 1 < A.Kw) store_a(buf ^ 1, ra);
      __syncthreads();
    }
  }
  const int xz = (A.xzp ? static_cast<int>(A.xzp[0]) : 0) - 128;
  const int32_t* xs = A.xs + b * A.Lp;
  const int64_t obase = b * A.Cout * A.Lout;
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int64_t l = nb + wn * (TN / 2) + 32 * ni + r;
    if (l >= A.Lout) continue;
    int S = 0;  // sum_k b_k of this output column
    for (int64_t tap = 0; tap < A.Kw; ++tap) S += xs[l * A.s + tap * A.d];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
      for (int reg = 0; reg < 16; ++reg) {
        const int64_t co = m0 + wm * 64 + 32 * mi + 8 * (reg / 4) + 4 * g + (reg % 4);
        if (co >= A.Cout) continue;
        const int wz = A.wzo[co];
        const int v = acc[mi][ni][reg] - xz * A.wsum[co] - wz * S +
                      static_cast<int>(A.Kreal) * wz * xz;
        if (A.outf) {
          const int vb = A.bias ? v + A.bias[co] : v;
          A.outf[obase + co * A.Lout + l] =
              static_cast<float>(vb) * A.scale[A.scale_n > 1 ? co : 0];
        } else {
          A.out[obase + co * A.Lout + l] = v;
        }
      }
    }
  }
}

}  // namespace

static int64_t conv_window(int64_t tn, int64_t stride, int64_t dilation, int64_t K) {
  return (tn - 1) * stride + (K - 1) * dilation + 1;
}

// The time tile (128, else 64) whose input window fits 64 KB of LDS beside
// the weight double buffer; 0 if neither does.
static int conv_tile_n(int64_t stride, int64_t dilation, int64_t K) {
  for (int tn : {128, 64})
    if (conv_window(tn, stride, dilation, K) * kRowPitch + 2 * kTileM * kRowPitch <= 65536)
      return tn;
  return 0;
}

// Shapes and zero points of ConvInteger (ref_runtime.py:130-134); fills
// *Lout.  Both zero points must be per tensor, as the reference reads them
// with np.int32(zp).
static int check_conv_integer(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                       const kk_tensor* x_zp, const kk_tensor* w_zp, int stride, int dilation,
                       int pad0, int pad1, int group, int out_dt, const char* who,
                       int64_t* lout) {
  KK_TRY(require_ready());
  KK_TRY(check_tensor(out, "out"));
  KK_TRY(check_tensor(x, "x"));
  KK_TRY(check_tensor(w, "w"));
  if (x->rank != 3 || w->rank != 3 || out->rank != 3)
    return set_error(KK_E_ARG, "%s: x, w and out must be rank 3", who);
  if (x->dtype != KK_U8 || !(w->dtype == KK_U8 || w->dtype == KK_I8) || out->dtype != out_dt)
    return set_error(KK_E_ARG, "%s: x uint8, w uint8/int8, out %s", who,
                     out_dt == KK_I32 ? "int32" : "fp32");
  if (!is_contiguous(x) || !is_contiguous(out) || !is_contiguous(w))
    return set_error(KK_E_ARG, "%s: x, w and out must be contiguous", who);
  if (group != 1) return set_error(KK_E_UNSUPPORTED, "%s: group %d", who, group);
  const int64_t N = x->shape[0], Cin = x->shape[1], L = x->shape[2];
  const int64_t Cout = w->shape[0], K = w->shape[2];
  if (w->shape[1] != Cin) return set_error(KK_E_ARG, "%s: w must be [Cout, Cin, K]", who);
  if (stride < 1 || dilation < 1 || pad0 < 0 || pad1 < 0)
    return set_error(KK_E_ARG, "%s: bad stride/dilation/pads", who);
  const int64_t span = static_cast<int64_t>(dilation) * (K - 1) + 1;
  const int64_t Lp = L + pad0 + pad1;
  const int64_t Lout = Lp >= span ? (Lp - span) / stride + 1 : 0;
  if (out->shape[0] != N || out->shape[1] != Cout || out->shape[2] != Lout)
    return set_error(KK_E_ARG, "%s: out must be [%lld, %lld, %lld]", who, (long long)N,
                     (long long)Cout, (long long)Lout);
  if (x_zp) {
    KK_TRY(check_tensor(x_zp, "x_zp"));
    if (x_zp->dtype != KK_U8 || numel(x_zp) != 1)
      return set_error(KK_E_ARG, "%s: x_zp must be one uint8", who);
  }
  if (w_zp) {
    KK_TRY(check_tensor(w_zp, "w_zp"));
    if (!(w_zp->dtype == KK_U8 || w_zp->dtype == KK_I8 || w_zp->dtype == KK_I32) ||
        numel(w_zp) != 1)
      return set_error(KK_E_ARG, "%s: w_zp must be one uint8/int8/int32", who);
  }
  // |each epilogue term| <= K * 2^14 must stay clear of 2^31.
  if (Cin * K > 32768)
    return set_error(KK_E_UNSUPPORTED, "%s: Cin*K = %lld exceeds 32768", who,
                     (long long)(Cin * K));
  if (N > 65535 || ceil_div(Lout, 64) > 0x7fffffff)
    return set_error(KK_E_UNSUPPORTED, "%s: grid too large", who);
  // a block's input window must fit LDS beside the weight double buffer
  if (conv_tile_n(stride, dilation, K) == 0)
    return set_error(KK_E_UNSUPPORTED, "%s: stride %d / dilation %d / kernel %lld: input window "
                     "of %lld rows does not fit LDS", who, stride, dilation, (long long)K,
                     (long long)conv_window(64, stride, dilation, K));
  *lout = Lout;
  return KK_OK;
}

// Both entry points: `outf` set gives the scaled fp32 form.
static int conv_integer_run(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                     const kk_tensor* x_zp, const kk_tensor* w_zp, const kk_tensor* bias,
                     const kk_tensor* scale, int stride, int dilation, int pad0, int pad1,
                     bool outf) {
  const int64_t N = x->shape[0], Cin = x->shape[1], L = x->shape[2];
  const int64_t Cout = w->shape[0], Kw = w->shape[2];
  const int64_t Lp = L + pad0 + pad1;
  const int64_t Lout = out->shape[2];
  const int64_t CinP = ceil_div(Cin, kCinAlign) * kCinAlign;
  const int64_t CoutP = ceil_div(Cout, kTileM) * kTileM;
  auto up = [](int64_t n) { return ceil_div(n, 256) * 256; };
  const int64_t o_wT = 0, o_wsum = o_wT + up(CoutP * Kw * CinP);
  const int64_t o_wzo = o_wsum + up(CoutP * 4), o_xs = o_wzo + up(CoutP * 4);
  const int64_t o_xT = o_xs + up(N * Lp * 4), total = o_xT + up(N * Lp * CinP);
  void* ws = nullptr;
  KK_TRY(kk_alloc(static_cast<size_t>(total), &ws));
  char* base = static_cast<char*>(ws);
  int8_t* wT = reinterpret_cast<int8_t*>(base + o_wT);
  int32_t* wsum = reinterpret_cast<int32_t*>(base + o_wsum);
  int32_t* wzo = reinterpret_cast<int32_t*>(base + o_wzo);
  int32_t* xs = reinterpret_cast<int32_t*>(base + o_xs);
  int8_t* xT = reinterpret_cast<int8_t*>(base + o_xT);
  hipStream_t st = ctx().stream;
  hipLaunchKernelGGL(conv_i8_wprep, dim3(static_cast<unsigned>(CoutP)), dim3(256), 0, st, w->data,
                     w->dtype, w_zp ? w_zp->data : nullptr, w_zp ? w_zp->dtype : 0,
                     w_zp ? numel(w_zp) : 0, wT, wsum, wzo, Cout, Cin, Kw, CinP);
  int rc = check_launch("conv_i8_wprep");
  const uint8_t* xzp = x_zp ? static_cast<const uint8_t*>(x_zp->data) : nullptr;
  if (rc == KK_OK) {
    hipLaunchKernelGGL(conv_i8_xprep, dim3(static_cast<unsigned>(ceil_div(Lp, kPrepT)),
                                           static_cast<unsigned>(N)),
                       dim3(256), 0, st, static_cast<const uint8_t*>(x->data), xzp, xT, xs, Cin,
                       L, static_cast<int64_t>(pad0), Lp, CinP);
    rc = check_launch("conv_i8_xprep");
  }
  if (rc == KK_OK) {
    ConvI8Args A{};
    A.wT = wT; A.wsum = wsum; A.wzo = wzo; A.xT = xT; A.xs = xs; A.xzp = xzp;
    if (outf) {
      A.outf = static_cast<float*>(out->data);
      A.bias = bias ? static_cast<const int32_t*>(bias->data) : nullptr;
      A.scale = static_cast<const float*>(scale->data);
      A.scale_n = numel(scale);
    } else {
      A.out = static_cast<int32_t*>(out->data);
    }
    A.Cout = Cout; A.CinP = CinP; A.Kw = Kw; A.s = stride; A.d = dilation; A.Lp = Lp;
    A.Lout = Lout; A.Kreal = Cin * Kw;
    const int tn = conv_tile_n(stride, dilation, Kw);
    A.W = static_cast<int>(conv_window(tn, stride, dilation, Kw));
    const size_t lds = static_cast<size_t>(A.W) * kRowPitch + 2 * kTileM * kRowPitch;
    const dim3 grid(static_cast<unsigned>(ceil_div(Lout, tn)),
                    static_cast<unsigned>(CoutP / kTileM), static_cast<unsigned>(N));
    if (tn == 128) hipLaunchKernelGGL(conv_i8_kernel<128>, grid, dim3(256), lds, st, A);
    else hipLaunchKernelGGL(conv_i8_kernel<64>, grid, dim3(256), lds, st, A);
    rc = check_launch("conv_i8_kernel");
  }
  kk_free(ws);  // stream order keeps the workspace alive for the kernels
  return rc;
}

}  // namespace kk

using namespace kk;

extern "C" {

int kk_conv_integer(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                    const kk_tensor* x_zp, const kk_tensor* w_zp, int stride, int dilation,
                    int pad0, int pad1, int group) {
  int64_t Lout = 0;
  KK_TRY(check_conv_integer(out, x, w, x_zp, w_zp, stride, dilation, pad0, pad1, group, KK_I32,
                            "kk_conv_integer", &Lout));
  if (numel(out) == 0) return KK_OK;
  if (x->shape[1] * w->shape[2] == 0) return kk_fill(out, 0.0);
  return conv_integer_run(out, x, w, x_zp, w_zp, nullptr, nullptr, stride, dilation, pad0, pad1,
                          false);
}

int kk_conv_integer_scaled(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                           const kk_tensor* x_zp, const kk_tensor* w_zp, const kk_tensor* bias,
                           const kk_tensor* scale, int stride, int dilation, int pad0, int pad1,
                           int group) {
  int64_t Lout = 0;
  KK_TRY(check_conv_integer(out, x, w, x_zp, w_zp, stride, dilation, pad0, pad1, group, KK_F32,
                            "kk_conv_integer_scaled", &Lout));
  const int64_t Cout = w->shape[0];
  KK_TRY(check_tensor(scale, "scale"));
  if (scale->dtype != KK_F32 || !is_contiguous(scale) ||
      (numel(scale) != 1 && numel(scale) != Cout))
    return set_error(KK_E_ARG, "kk_conv_integer_scaled: scale must be fp32 with 1 or Cout values");
  if (bias) {
    KK_TRY(check_tensor(bias, "bias"));
    if (bias->dtype != KK_I32 || !is_contiguous(bias) || numel(bias) != Cout)
      return set_error(KK_E_ARG, "kk_conv_integer_scaled: bias must be int32 with Cout values");
  }
  if (numel(out) == 0) return KK_OK;
  if (x->shape[1] * w->shape[2] == 0)
    return set_error(KK_E_UNSUPPORTED, "kk_conv_integer_scaled: empty reduction");
  return conv_integer_run(out, x, w, x_zp, w_zp, bias, scale, stride, dilation, pad0, pad1, true);
}

}  // extern "C"
