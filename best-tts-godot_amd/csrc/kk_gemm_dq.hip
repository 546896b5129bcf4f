// MatMul of fp32 activations with 8-bit weights on the bf16 matrix cores,
// with the accuracy of fp32 products accumulated in fp32:
//
//   out[m, n] = alpha * s[n] * sum_k A[m, k] * (q[k, n] - z[n])
//
// Exact operands:
//  * an 8-bit weight less its zero point of the same type is an integer of
//    at most 255 in magnitude: 8 significant bits, exact in bf16;
//  * an fp32 activation is a0 + a1 + a2: a0 = a with the low 16 bits of its
//    encoding cleared, r = a - a0 (exact: the low 16 bits of the
//    significand), a1 = r with its low 16 bits cleared, a2 = r - a1 (exact,
//    at most 8 significant bits).  Truncation never overflows and bf16 has
//    fp32's exponent range, so no scaling is needed whatever the
//    activations' magnitude (only fp32 subnormals below 2^-110 lose bits).
// Every product a_i * (q - z) is then exact in fp32, and three
// v_mfma_f32_32x32x16_bf16 per product accumulate them in fp32.  The scale
// (per tensor or per column) multiplies the fp32 sum, where the numpy
// reference scales each weight first: the same value up to fp32 rounding.
// For a = +-inf, a0 = a and a1 = a2 = 0; a NaN gives NaN parts.
//
// Two launches.  gemm_dq_prep writes the operands once, into the library
// scratch: A as three bf16 planes [3][Mp][Kp] and B as bf16 [Np][Kp],
// transposed so that k is contiguous for both (Mp, Np, Kp: M, N, K rounded
// up to the largest tile, zero-filled).  Splitting inside the GEMM instead
// repeated the split for every block column (and B's conversion for every
// block row) and left the kernel VALU-bound at 4-5x its matrix-core time.
// gemm_bf16_kernel is then a plain bf16 GEMM: a block of four waves, each
// owning one 32x32 output tile and a k-slice of 32 of each staged K-step
// (Shape<WM, WN, KS>: (32 WM) x (32 WN) outputs, KS k-slices,
// WM * WN * KS = 4), whose partial tiles are summed through LDS in slice
// order; the global loads of the next kRing K-steps are in flight in
// registers while a step is multiplied.  Splitting K over blocks as well
// (the last block of a tile to arrive summing the partial tiles) measured
// slower at every split count tried: at M = 256 the partials' round trip
// through the device-coherent level costs more than the added blocks gain.
// fp16 weights (two bf16 planes, five MFMAs per product) were measured on
// this path too and were slower than the fp32 matrix cores at
// 256 x 768 x 768 (16.5 vs 15.2 us): they stay there.
#include <algorithm>
#include <type_traits>

#include "kk_internal.h"

namespace kk {
namespace gdq {

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kRing = 4;  // K-steps whose global loads are in flight ahead of use
constexpr int kPadM = 64, kPadN = 64, kPadK = 128;  // prepared operand padding (largest tile)

// ------------------------------------------------------------- operand prep
// a = a0 + a1 + a2 (see the top of the file): each part's bf16 bits are the
// upper half of the returned word (the lower half is not used).
__device__ __forceinline__ void split3(float a, unsigned& h0, unsigned& h1, unsigned& h2) {
  const unsigned u = __float_as_uint(a);
  const float a0 = __uint_as_float(u & 0xffff0000u);
  const float r = a0 == a ? 0.0f : a - a0;
  const unsigned ur = __float_as_uint(r);
  h0 = u;
  h1 = ur;
  h2 = __float_as_uint(r - __uint_as_float(ur & 0xffff0000u));
}

// The upper halves of lo and hi as two packed bf16 (lo first).
__device__ __forceinline__ unsigned pack_hi(unsigned lo, unsigned hi) {
  return __builtin_amdgcn_perm(hi, lo, 0x07060302u);
}

struct PrepArgs {
  const float* a;  // A [M, K] rows a_si apart, K contiguous (K % 4 == 0, 16-byte aligned rows)
  int64_t a_si;
  const void* b;   // B [K, N] rows b_si apart, N contiguous (N % 4 == 0)
  int64_t b_si;
  int b_dt;        // KK_I8 or KK_U8
  const void* zp;  // zero point (same type as B) or NULL
  int64_t zp_stride;
  __bf16* ap;      // [3][Mp][Kp]
  __bf16* bp;      // [Np][Kp]
  int64_t M, N, K, Mp, Np, Kp;
  int a_blocks;    // blocks [0, a_blocks) split A; the rest convert B tiles of 64 k x 64 n
};

constexpr int kPrepQuads = 4;  // A quads (4 k) per thread
constexpr int kTileRow = 64 * 2 + 16;  // LDS bytes per n row of a B tile: 64 k of 2 bytes, padded

__global__ void __launch_bounds__(256) gemm_dq_prep(PrepArgs P) {
  __shared__ __align__(16) unsigned char tile[64 * kTileRow];  // [n][k], 2 bytes per k
  const int tid = threadIdx.x;
  if (static_cast<int>(blockIdx.x) < P.a_blocks) {
    const int64_t kq = P.Kp / 4;
#pragma unroll
    for (int j = 0; j < kPrepQuads; ++j) {
      const int64_t q = (static_cast<int64_t>(blockIdx.x) * kPrepQuads + j) * 256 + tid;
      if (q >= P.Mp * kq) return;
      const int64_t m = q / kq, k = (q - m * kq) * 4;
      float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (m < P.M && k < P.K) v = *reinterpret_cast<const float4*>(P.a + m * P.a_si + k);
      unsigned h[3][4];
      split3(v.x, h[0][0], h[1][0], h[2][0]);
      split3(v.y, h[0][1], h[1][1], h[2][1]);
      split3(v.z, h[0][2], h[1][2], h[2][2]);
      split3(v.w, h[0][3], h[1][3], h[2][3]);
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
        *reinterpret_cast<uint2*>(P.ap + (pl * P.Mp + m) * P.Kp + k) =
            make_uint2(pack_hi(h[pl][0], h[pl][1]), pack_hi(h[pl][2], h[pl][3]));
    }
    return;
  }
  // a B tile: k0..k0+63 x n0..n0+63, read n-contiguous, written k-contiguous
  const int64_t bt = blockIdx.x - P.a_blocks, ntn = P.Np / 64;
  const int64_t k0 = (bt / ntn) * 64, n0 = (bt % ntn) * 64;
  // stage: thread -> k rows tid / 16 + 16 j, n quad tid % 16; each weight
  // goes to its [n][k] slot widened to 2 bytes
  {
    const int nq = tid % 16;
    const int64_t n = n0 + 4 * nq;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kr = tid / 16 + 16 * j;
      const int64_t k = k0 + kr;
      const bool in = k < P.K && n < P.N;  // N % 4 == 0: four columns or none
      // outside K: the zero point itself, so that q - zp = 0 there
      unsigned u = 0u;
      if (in) {
        u = *reinterpret_cast<const unsigned*>(static_cast<const uint8_t*>(P.b) + k * P.b_si + n);
      } else if (P.zp && n < P.N) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          u |= static_cast<unsigned>(static_cast<const uint8_t*>(P.zp)[(n + c) * P.zp_stride])
               << (8 * c);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *reinterpret_cast<unsigned short*>(&tile[(4 * nq + c) * kTileRow + 2 * kr]) =
            static_cast<unsigned short>((u >> (8 * c)) & 0xffu);
    }
  }
  __syncthreads();
  // write: thread -> n row tid / 4, k values 16 (tid % 4) .. + 15
  const int nr = tid / 4, kc = 16 * (tid % 4);
  const int64_t n = n0 + nr;
  const uint4* src = reinterpret_cast<const uint4*>(&tile[nr * kTileRow + 2 * kc]);
  const uint4 s0 = src[0], s1 = src[1];
  const unsigned w[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  __bf16* out0 = P.bp + n * P.Kp + k0 + kc;
  const bool i8 = P.b_dt == KK_I8;
  float z = 0.0f;
  if (P.zp && n < P.N) {
    const uint8_t zb = static_cast<const uint8_t*>(P.zp)[n * P.zp_stride];
    z = i8 ? static_cast<float>(static_cast<int8_t>(zb)) : static_cast<float>(zb);
  }
  unsigned p[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    unsigned h[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const unsigned byte = (w[i] >> (16 * e)) & 0xffu;
      const float q = i8 ? static_cast<float>(static_cast<int8_t>(byte)) : static_cast<float>(byte);
      h[e] = __float_as_uint(q - z);  // an integer of magnitude <= 255: exact in bf16
    }
    p[i] = n < P.N ? pack_hi(h[0], h[1]) : 0u;  // padding columns: zeros
  }
  reinterpret_cast<uint4*>(out0)[0] = make_uint4(p[0], p[1], p[2], p[3]);
  reinterpret_cast<uint4*>(out0)[1] = make_uint4(p[4], p[5], p[6], p[7]);
}

// ------------------------------------------------------------------- GEMM
template <int WM_, int WN_, int KS_>
struct Shape {
  static constexpr int WM = WM_, WN = WN_, KS = KS_;
  static constexpr int BM = 32 * WM, BN = 32 * WN, BK = 32 * KS;
  static constexpr int P = BK + 8;    // LDS row pitch (bf16): conflict-free 16-byte reads
  static constexpr int CPR = BK / 8;  // 16-byte chunks per row of a K-step
  static_assert(WM * WN * KS == 4, "four waves");
  static_assert(kPadK % BK == 0 && kPadM % BM == 0 && kPadN % BN == 0,
                "the padding covers the tiles");
};

struct Args {
  const __bf16* ap;   // [3][Mp][Kp]
  const __bf16* bp;   // [Np][Kp]
  const void* scale;  // per tensor or per column
  int scale_dt;
  int64_t scale_stride;
  float* out;
  int64_t som, son;
  int64_t M, N, Mp, Np, Kp;
  float alpha;
};

template <class S>
__global__ void __launch_bounds__(kThreads) gemm_bf16_kernel(Args G) {
  constexpr int P = S::P;
  constexpr int AC = 3 * S::BM * S::CPR / kThreads;   // A chunks per thread per step
  constexpr int BC = S::BN * S::CPR / kThreads;       // B chunks per thread per step
  static_assert(AC * kThreads == 3 * S::BM * S::CPR && BC * kThreads == S::BN * S::CPR,
                "staging shape");
  __shared__ __align__(16) __bf16 As[2][3 * S::BM * P];
  __shared__ __align__(16) __bf16 Bs[2][S::BN * P];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ks = wave / (S::WM * S::WN), wt = wave % (S::WM * S::WN);
  const int wmi = wt / S::WN, wni = wt % S::WN;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * S::BM;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * S::BN;
  const int64_t Kp = G.Kp;
  const int nk = static_cast<int>(Kp / S::BK);  // K-steps (>= 1: Kp is a whole number of them)

  // staging: chunk c of this thread is row r (plane-major: plane r / BM,
  // row r % BM), 8 k from 8 * (c % CPR)
  const __bf16* asrc[AC];
  int adst[AC];
#pragma unroll
  for (int c = 0; c < AC; ++c) {
    const int idx = tid + c * kThreads, r = idx / S::CPR, ch = idx % S::CPR;
    const int pl = r / S::BM, m = r % S::BM;
    asrc[c] = G.ap + (pl * G.Mp + m0 + m) * Kp + 8 * ch;
    adst[c] = r * P + 8 * ch;
  }
  const __bf16* bsrc[BC];
  int bdst[BC];
#pragma unroll
  for (int c = 0; c < BC; ++c) {
    const int idx = tid + c * kThreads, r = idx / S::CPR, ch = idx % S::CPR;
    bsrc[c] = G.bp + (n0 + r) * Kp + 8 * ch;
    bdst[c] = r * P + 8 * ch;
  }

  u4 av[kRing][AC], bv[kRing][BC];
  auto fetch = [&](int sl, int kt) {  // past the end: the last step again (never used)
    const int64_t k0 = static_cast<int64_t>(kt < nk ? kt : nk - 1) * S::BK;
#pragma unroll
    for (int c = 0; c < AC; ++c) av[sl][c] = *reinterpret_cast<const u4*>(asrc[c] + k0);
#pragma unroll
    for (int c = 0; c < BC; ++c) bv[sl][c] = *reinterpret_cast<const u4*>(bsrc[c] + k0);
  };
  auto stash = [&](int sl, int buf) {
#pragma unroll
    for (int c = 0; c < AC; ++c) *reinterpret_cast<u4*>(&As[buf][adst[c]]) = av[sl][c];
#pragma unroll
    for (int c = 0; c < BC; ++c) *reinterpret_cast<u4*>(&Bs[buf][bdst[c]]) = bv[sl][c];
  };

  const int arow_l = (32 * wmi + (lane & 31)) * P, brow_l = (32 * wni + (lane & 31)) * P;
  constexpr int kPlaneA = S::BM * P;
  f16v acc;
#pragma unroll
  for (int g = 0; g < 16; ++g) acc[g] = 0.0f;
  auto multiply = [&](int buf) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int kofs = 32 * ks + 16 * c + 8 * (lane >> 5);
      const bf8 a0 = *reinterpret_cast<const bf8*>(&As[buf][arow_l + kofs]);
      const bf8 a1 = *reinterpret_cast<const bf8*>(&As[buf][kPlaneA + arow_l + kofs]);
      const bf8 a2 = *reinterpret_cast<const bf8*>(&As[buf][2 * kPlaneA + arow_l + kofs]);
      const bf8 b0 = *reinterpret_cast<const bf8*>(&Bs[buf][brow_l + kofs]);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, b0, acc, 0, 0, 0);
    }
  };

  // Step kt: stash the next step from its slot into the other LDS buffer and
  // refill that slot kRing steps ahead, multiply this step, one barrier.
  fetch(0, 0);
  fetch(1, 1);
  fetch(2, 2);
  fetch(3, 3);
  stash(0, 0);
  if (kRing < nk) fetch(0, kRing);
  __syncthreads();
  // one step with its ring slots as constants (the ring stays in registers)
  auto step = [&](auto uc, int kt) {
    constexpr int u = decltype(uc)::value;
    if (kt + 1 < nk) stash((u + 1) % kRing, (u & 1) ^ 1);
    if (kt + 1 + kRing < nk) fetch((u + 1) % kRing, kt + 1 + kRing);  // (kt is uniform)
    multiply(u & 1);
    __syncthreads();
  };
  static_assert(kRing == 4, "the loop below is written out for four slots");
  for (int t = 0; t < nk; t += kRing) {
    step(std::integral_constant<int, 0>{}, t);
    if (t + 1 >= nk) break;
    step(std::integral_constant<int, 1>{}, t + 1);
    if (t + 2 >= nk) break;
    step(std::integral_constant<int, 2>{}, t + 2);
    if (t + 3 >= nk) break;
    step(std::integral_constant<int, 3>{}, t + 3);
  }

  // k-slices 1.. hand their partial tiles to slice 0 through LDS (the
  // staging buffers are free after the last barrier); slice 0 adds them in
  // slice order
  if constexpr (S::KS > 1) {
    static_assert((S::KS - 1) * S::WM * S::WN * 1024 * 4 <= sizeof(As), "reduction space");
    float* red = reinterpret_cast<float*>(&As[0][0]);
    if (ks > 0) {
      float* dst = red + ((ks - 1) * S::WM * S::WN + wt) * 1024;
#pragma unroll
      for (int g = 0; g < 16; ++g) dst[g * 64 + lane] = acc[g];
    }
    __syncthreads();
    if (ks == 0) {
#pragma unroll
      for (int s = 1; s < S::KS; ++s) {
        const float* src = red + ((s - 1) * S::WM * S::WN + wt) * 1024;
#pragma unroll
        for (int g = 0; g < 16; ++g) acc[g] += src[g * 64 + lane];
      }
    }
  }

  if (ks > 0) return;

  // D(i, j) of a 32x32 tile: lane j + 32 * ((i / 4) % 2), register (i / 8) * 4 + i % 4
  const int64_t n = n0 + 32 * wni + (lane & 31);
  if (n >= G.N) return;
  const float sc = load_as_f32(G.scale, G.scale_dt, n * G.scale_stride);
  float* o = G.out + n * G.son;
  const float alpha = G.alpha;
#pragma unroll
  for (int g = 0; g < 16; ++g) {
    const int64_t m = m0 + 32 * wmi + 8 * (g / 4) + 4 * (lane >> 5) + (g % 4);
    if (m >= G.M) continue;
    float v = acc[g] * sc;
    if (alpha != 1.0f) v *= alpha;
    o[m * G.som] = v;
  }
}

}  // namespace gdq

// Runs out = A @ dequant(B) on the bf16 matrix cores when the operands fit
// (see the top of the file); returns false, launching nothing, otherwise:
// A fp32 with K contiguous (K % 4 == 0, 16-byte aligned rows), B int8/uint8
// (zero point of the same type or none) or fp16 with N contiguous and
// N % 4 == 0; batch axes only where B is shared and A and out are whole
// [batch * M] row ranges; the prepared operands within the scratch.
bool gemm_dq_try(const float* a, int64_t a_si, const void* b, int b_dt, int64_t b_si,
                 const Dequant& dq, float* out, int64_t som, int64_t son, const BatchMap& bm,
                 int64_t M, int64_t N, int64_t K, int64_t batch, float alpha, const int* only_if,
                 int* status) {
  using namespace gdq;
  *status = KK_OK;
  if (only_if) return false;
  if (!(b_dt == KK_I8 || b_dt == KK_U8)) return false;
  if (!dq.active || !dq.scale || (dq.zp && dq.zp_dt != b_dt)) return false;
  if (K % 4 || a_si % 4 || (reinterpret_cast<uintptr_t>(a) & 15)) return false;
  if (N % 4 || b_si % 4 || (reinterpret_cast<uintptr_t>(b) & 3)) return false;
  // batch axes: B shared; A and out rows of consecutive batches follow on
  int64_t ea = M * a_si, eo = M * som;
  for (int d = bm.nb - 1; d >= 0; --d) {
    if (bm.dims[d] == 1) continue;
    if (bm.st[1][d] != 0 || bm.st[0][d] != ea || bm.st[2][d] != eo) return false;
    ea *= bm.dims[d];
    eo *= bm.dims[d];
  }
  const int64_t Mt = M * batch;  // A and out as [batch * M] rows
  const int64_t Mp = ceil_div(Mt, kPadM) * kPadM, Np = ceil_div(N, kPadN) * kPadN,
                Kp = ceil_div(K, kPadK) * kPadK;
  const size_t a_bytes = static_cast<size_t>(3 * Mp * Kp) * 2;
  const size_t b_bytes = static_cast<size_t>(Np * Kp) * 2;
  if (a_bytes + b_bytes > kScratchBytes || ceil_div(Mt, 32) > 65535 ||
      ceil_div(N, 32) > (int64_t{1} << 30))
    return false;

  char* scratch = static_cast<char*>(ctx().scratch);
  PrepArgs pa{a, a_si, b, b_si, b_dt, dq.zp, dq.zp_stride,
              reinterpret_cast<__bf16*>(scratch), reinterpret_cast<__bf16*>(scratch + a_bytes),
              Mt, N, K, Mp, Np, Kp, 0};
  pa.a_blocks = static_cast<int>(ceil_div(Mp * (Kp / 4), 256 * kPrepQuads));
  const int64_t b_blocks = (Kp / 64) * (Np / 64);
  hipLaunchKernelGGL(gemm_dq_prep, dim3(static_cast<unsigned>(pa.a_blocks + b_blocks)), dim3(256), 0,
                     ctx().stream, pa);
  *status = check_launch("gemm_dq_prep");
  if (*status != KK_OK) return true;

  const Args g{pa.ap, pa.bp, dq.scale, dq.scale_dt, dq.scale_stride, out, som, son, Mt, N, Mp, Np,
               Kp, alpha};
  // The largest output tile whose blocks still cover every CU, else the
  // smallest (32 x 32, K split over the four waves).
  const int64_t cus = ctx().num_cus > 0 ? ctx().num_cus : 256;
  auto tiles = [&](int bm_, int bn_) { return ceil_div(Mt, bm_) * ceil_div(N, bn_); };
  const int shape = tiles(64, 64) >= cus ? 0 : tiles(32, 64) >= cus ? 1 : 2;
#define KK_DQ_LAUNCH(SH)                                                                    \
  hipLaunchKernelGGL((gemm_bf16_kernel<SH>),                                                \
                     dim3(static_cast<unsigned>(ceil_div(N, SH::BN)),                       \
                          static_cast<unsigned>(ceil_div(Mt, SH::BM))),                     \
                     dim3(kThreads), 0, ctx().stream, g)
  using S64x64 = Shape<2, 2, 1>;
  using S32x64 = Shape<1, 2, 2>;
  using S32x32 = Shape<1, 1, 4>;
  if (shape == 0) KK_DQ_LAUNCH(S64x64);
  else if (shape == 1) KK_DQ_LAUNCH(S32x64);
  else KK_DQ_LAUNCH(S32x32);
#undef KK_DQ_LAUNCH
  *status = check_launch("gemm_bf16_kernel");
  return true;
}

}  // namespace kk
