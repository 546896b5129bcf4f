// MatMul of fp32 activations with 8-bit or fp16 weights on the bf16 matrix
// cores, with the accuracy of fp32 products accumulated in fp32:
//
//   out[m, n] = alpha * s[n] * sum_k A[m, k] * (q[k, n] - z[n])   (8-bit)
//   out[m, n] = alpha * sum_k A[m, k] * B[k, n]                   (fp16)
//
// Exact operands:
//  * an 8-bit weight less its zero point of the same type is an integer of
//    at most 255 in magnitude: 8 significant bits, exact in bf16;
//  * an fp16 weight has at most 11 significant bits and lies within bf16's
//    exponent range: b = b0 + b1 with b0 = b with the low 16 bits of its
//    fp32 encoding cleared and b1 = b - b0 (at most 3 significant bits),
//    both exact in bf16;
//  * an fp32 activation is a0 + a1 + a2: a0 = a with the low 16 bits of its
//    encoding cleared, r = a - a0 (exact: the low 16 bits of the
//    significand), a1 = r with its low 16 bits cleared, a2 = r - a1 (exact,
//    at most 8 significant bits).  Truncation never overflows and bf16 has
//    fp32's exponent range, so no scaling is needed whatever the
//    activations' magnitude (only fp32 subnormals below 2^-110 lose bits).
// Every product a_i * b_j is then exact in fp32, and one
// v_mfma_f32_32x32x16_bf16 per pair of parts (three for 8-bit weights, six
// for fp16) accumulates them in fp32.  The scale (per tensor or per column)
// multiplies the fp32 sum, where the numpy reference scales each weight
// first: the same value up to fp32 rounding.  For a = +-inf, a0 = a and
// a1 = a2 = 0 (likewise for b); a NaN gives NaN parts.  With 8-bit weights
// that reproduces numpy's inf and NaN outputs (inf * (q - z) is inf, or NaN
// at q = z, as in numpy); with fp16 weights a part of 0 meets an infinite
// one (a0 * b1 with b1 = 0), which gives NaN where numpy has +-inf.  So the
// fp16 prep stamps a flag with the call's number when any operand is not
// finite, and a block that finds its call's stamp computes its tile with
// scalar fp32 products of the reassembled operands (a0 + a1 + a2 and
// b0 + b1 are a and b exactly, infinities and NaN included) instead.  A
// stale stamp (a recorded graph replays its calls' numbers) only costs that
// slower path.
//
// Two launches.  gemm_dq_prep writes the operands once, into the library
// scratch: A as three bf16 planes and B as one or two, each of Mp x Kp
// (Np x Kp) values (M, N, K rounded up to the padding below, zero-filled;
// 8-bit B is filled with its zero point past K), in fragment order: the
// values of rows 32 t .. 32 t + 31 and K-step s (k = 32 s .. 32 s + 31) are
// two fragments of 64 lanes x 8 bf16 (half h), lane l holding row
// 32 t + l % 32 at k = 32 s + 16 (l / 32) + 8 h + 0..7, so that one
// 16-byte load per lane is its share of a matrix-core operand (row =
// lane % 32, 8 consecutive k) and a wave's load is 1 KB of consecutive
// bytes.  Splitting inside the GEMM instead repeated the split for every
// block column (and B's conversion for every block row) and left the
// kernel VALU-bound at 4-5x its matrix-core time.
//
// gemm_bf16_kernel: every wave loads its fragments straight into
// registers, with no LDS staging and no barrier in the K loop (with the
// operands row-major instead, each load touched 32 rows and the kernel was
// slower than the staged one).  A block of KS waves owns a 32 x (32 NT) output tile; wave w takes
// the w-th of KS consecutive runs of 32-wide K-steps, keeps the loads of its
// next RING steps in flight in a register ring and accumulates into 2 NT
// independent 32x32 tiles (one per half of each K-step, so consecutive
// matrix-core operations do not wait on one another).  At the end the
// waves hand their partial tiles through LDS and each sums a share of the
// tile in wave order and writes it.  An earlier form staged both operands
// through LDS with a barrier per K-step and one accumulator per wave: at
// 256 x 768 x 2048 its waves spent half their time waiting (10.0 us).
// Splitting K over blocks as well (the last block of a tile to arrive
// summing the partial tiles) measured slower: at M = 256 the partials'
// round trip through the device-coherent level costs more than the added
// blocks gain.
#include <algorithm>
#include <type_traits>

#include "kk_internal.h"

namespace kk {
namespace gdq {

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));

constexpr int kPadM = 64, kPadN = 64, kPadK = 128;  // prepared operand padding

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

// Offset (in bf16) of the 8-value lane chunk of fragment (row tile t,
// K-step s, half h), lane l, within a plane of nk K-steps.
__device__ __forceinline__ int64_t frag_chunk(int64_t t, int64_t s, int h, int l, int64_t nk) {
  return ((t * nk + s) * 2 + h) * 512 + l * 8;
}

// Offset of value (row, k) within a plane of nk K-steps.
__device__ __forceinline__ int64_t frag_index(int64_t row, int64_t k, int64_t nk) {
  const int kk = static_cast<int>(k & 31);
  return frag_chunk(row >> 5, k >> 5, (kk >> 3) & 1, static_cast<int>(row & 31) + 32 * (kk >> 4),
                    nk) +
         (kk & 7);
}

struct PrepArgs {
  const float* a;  // A [M, K] rows a_si apart, K contiguous (K % 4 == 0, 16-byte aligned rows)
  int64_t a_si;
  const void* b;   // B [K, N] rows b_si apart, N contiguous (N % 4 == 0)
  int64_t b_si;
  int b_dt;        // KK_I8, KK_U8 or KK_F16
  const void* zp;  // zero point (same type as 8-bit B) or NULL
  int64_t zp_stride;
  __bf16* ap;      // 3 planes of Mp x Kp, fragment order
  __bf16* bp;      // BP planes of Np x Kp, fragment order (BP = 2 for fp16 B, else 1)
  int64_t M, N, K, Mp, Np, Kp;
  int a_blocks;    // blocks [0, a_blocks) split A (a lane chunk per thread); the rest
                   // convert B tiles of 64 k x 64 n
  int* flag;       // fp16 B: set to seq when an operand is not finite; else NULL
  int seq;
};

__device__ __forceinline__ bool f32_nonfinite(float x) {
  return (__float_as_uint(x) & 0x7f800000u) == 0x7f800000u;
}

constexpr int kTileRow = 64 * 2 + 16;  // LDS bytes per n row of a B tile: 64 k of 2 bytes, padded

__global__ void __launch_bounds__(256) gemm_dq_prep(PrepArgs P) {
  __shared__ __align__(16) unsigned char tile[64 * kTileRow];  // [n][k], 2 bytes per k
  const int tid = threadIdx.x;
  if (static_cast<int>(blockIdx.x) < P.a_blocks) {
    // thread -> lane chunk q: lane q % 64, half (q / 64) % 2, K-step
    // (q / 128) % nk, row tile q / (128 nk); each plane's chunk is written
    // whole, so a wave writes 1 KB of consecutive bytes per plane
    const int64_t nk = P.Kp / 32;
    const int64_t q = static_cast<int64_t>(blockIdx.x) * 256 + tid;
    if (q >= P.Mp * P.Kp / 8) return;
    const int l = static_cast<int>(q & 63), h = static_cast<int>((q >> 6) & 1);
    const int64_t st = q >> 7, s = st % nk, t = st / nk;
    const int64_t m = 32 * t + (l & 31), k = 32 * s + 16 * (l >> 5) + 8 * h;
    float v[8];
#pragma unroll
    for (int e = 0; e < 2; ++e) {  // K % 4 == 0: four values or none
      float4 x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (m < P.M && k + 4 * e < P.K)
        x = *reinterpret_cast<const float4*>(P.a + m * P.a_si + k + 4 * e);
      v[4 * e] = x.x;
      v[4 * e + 1] = x.y;
      v[4 * e + 2] = x.z;
      v[4 * e + 3] = x.w;
    }
    unsigned hp[3][8];
    bool bad = false;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      bad |= f32_nonfinite(v[e]);
      split3(v[e], hp[0][e], hp[1][e], hp[2][e]);
    }
    if (P.flag && bad) *P.flag = P.seq;  // every writer stores the same value
    const int64_t off = frag_chunk(t, s, h, l, nk);
#pragma unroll
    for (int pl = 0; pl < 3; ++pl)
      *reinterpret_cast<uint4*>(P.ap + pl * P.Mp * P.Kp + off) =
          make_uint4(pack_hi(hp[pl][0], hp[pl][1]), pack_hi(hp[pl][2], hp[pl][3]),
                     pack_hi(hp[pl][4], hp[pl][5]), pack_hi(hp[pl][6], hp[pl][7]));
    return;
  }
  // a B tile: k0..k0+63 x n0..n0+63, read n-contiguous, written k-contiguous
  const int64_t bt = blockIdx.x - P.a_blocks, ntn = P.Np / 64;
  const int64_t k0 = (bt / ntn) * 64, n0 = (bt % ntn) * 64;
  const bool f16 = P.b_dt == KK_F16;
  // stage: thread -> k rows tid / 16 + 16 j, n quad tid % 16; each weight's
  // raw bits (a byte zero-extended, or the fp16 encoding) go to its [n][k]
  // slot
  {
    const int nq = tid % 16;
    const int64_t n = n0 + 4 * nq;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kr = tid / 16 + 16 * j;
      const int64_t k = k0 + kr;
      const bool in = k < P.K && n < P.N;  // N % 4 == 0: four columns or none
      unsigned short e[4] = {0, 0, 0, 0};
      if (f16) {
        if (in) {
          const uint2 u =
              *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(P.b) + k * P.b_si + n);
          e[0] = static_cast<unsigned short>(u.x & 0xffffu);
          e[1] = static_cast<unsigned short>(u.x >> 16);
          e[2] = static_cast<unsigned short>(u.y & 0xffffu);
          e[3] = static_cast<unsigned short>(u.y >> 16);
          if ((e[0] & 0x7c00u) == 0x7c00u || (e[1] & 0x7c00u) == 0x7c00u ||
              (e[2] & 0x7c00u) == 0x7c00u || (e[3] & 0x7c00u) == 0x7c00u)
            *P.flag = P.seq;  // an fp16 inf or NaN (every writer stores the same value)
        }
      } else {
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
        for (int c = 0; c < 4; ++c) e[c] = static_cast<unsigned short>((u >> (8 * c)) & 0xffu);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *reinterpret_cast<unsigned short*>(&tile[(4 * nq + c) * kTileRow + 2 * kr]) = e[c];
    }
  }
  __syncthreads();
  // write: thread -> n row tid / 4, k values 16 (tid % 4) .. + 15: the
  // chunks of halves 0 and 1 of lane n % 32 + 32 (tid % 2) in K-step
  // (k0 + 16 (tid % 4)) / 32
  const int nr = tid / 4, c = tid % 4, kc = 16 * c;
  const int64_t n = n0 + nr;
  const uint4* src = reinterpret_cast<const uint4*>(&tile[nr * kTileRow + 2 * kc]);
  const uint4 s0 = src[0], s1 = src[1];
  const unsigned w[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  const int64_t nkb = P.Kp / 32;
  __bf16* out0 = P.bp + frag_chunk(n >> 5, (k0 + kc) >> 5, 0, static_cast<int>(n & 31) + 32 * (c & 1),
                                   nkb);
  __bf16* out0h = out0 + 512;  // half 1 of the same lane
  unsigned p[8], p1[8];
  if (f16) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      unsigned h0[2], h1[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const unsigned short bits = static_cast<unsigned short>((w[i] >> (16 * e)) & 0xffffu);
        const float b = static_cast<float>(__builtin_bit_cast(_Float16, bits));  // exact
        const float b0 = __uint_as_float(__float_as_uint(b) & 0xffff0000u);
        h0[e] = __float_as_uint(b);
        h1[e] = __float_as_uint(b0 == b ? 0.0f : b - b0);  // <= 3 significant bits: exact
      }
      p[i] = pack_hi(h0[0], h0[1]);
      p1[i] = pack_hi(h1[0], h1[1]);
    }
  } else {
    const bool i8 = P.b_dt == KK_I8;
    float z = 0.0f;
    if (P.zp && n < P.N) {
      const uint8_t zb = static_cast<const uint8_t*>(P.zp)[n * P.zp_stride];
      z = i8 ? static_cast<float>(static_cast<int8_t>(zb)) : static_cast<float>(zb);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      unsigned h[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const unsigned byte = (w[i] >> (16 * e)) & 0xffu;
        const float q =
            i8 ? static_cast<float>(static_cast<int8_t>(byte)) : static_cast<float>(byte);
        h[e] = __float_as_uint(q - z);  // an integer of magnitude <= 255: exact in bf16
      }
      p[i] = n < P.N ? pack_hi(h[0], h[1]) : 0u;  // padding columns: zeros
      p1[i] = 0u;
    }
  }
  *reinterpret_cast<uint4*>(out0) = make_uint4(p[0], p[1], p[2], p[3]);
  *reinterpret_cast<uint4*>(out0h) = make_uint4(p[4], p[5], p[6], p[7]);
  if (f16) {
    const int64_t pl = P.Np * P.Kp;
    *reinterpret_cast<uint4*>(out0 + pl) = make_uint4(p1[0], p1[1], p1[2], p1[3]);
    *reinterpret_cast<uint4*>(out0h + pl) = make_uint4(p1[4], p1[5], p1[6], p1[7]);
  }
}

// ------------------------------------------------------------------- GEMM
// NT 32-wide column tiles per block, KS waves splitting K, BP planes of B.
template <int NT_, int KS_, int BP_>
struct Shape {
  static constexpr int NT = NT_, KS = KS_, BP = BP_;
  static constexpr int BN = 32 * NT, THREADS = 64 * KS;
  // 16-byte loads per lane per 32-wide K-step: two halves of 3 A planes and
  // of BP B planes per column tile
  static constexpr int LOADS = 2 * (3 + BP * NT);
  static constexpr int RING = LOADS * 4 <= 40 ? 4 : 3;  // K-steps in flight (<= 42 loads)
  static constexpr int SHARE = NT * 16 / KS;             // output registers each wave sums
  static_assert(kPadN % BN == 0 && kPadK % 32 == 0, "the padding covers the tiles");
  static_assert(SHARE * KS == NT * 16, "the tile's registers divide over the waves");
};

struct Args {
  const __bf16* ap;   // 3 planes of Mp x Kp, fragment order
  const __bf16* bp;   // BP planes of Np x Kp, fragment order
  const void* scale;  // per tensor or per column, or NULL (1)
  int scale_dt;
  int64_t scale_stride;
  float* out;
  int64_t som, son;
  int64_t M, N, Mp, Np, Kp;
  float alpha;
  const int* flag;  // fp16 B: equal to seq when an operand of this call is not finite
  int seq;
};

// The tile of block (blockIdx.x, blockIdx.y) with scalar fp32 products of
// the reassembled operands (a = a0 + a1 + a2 and b = b0 + b1 exactly),
// summed in k order: numpy's results for infinite and NaN operands.
template <class S>
__device__ void exact_tile(const Args& G) {
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * 32;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * S::BN;
  const int64_t a_pl = G.Mp * G.Kp, b_pl = G.Np * G.Kp;
  for (int e = threadIdx.x; e < 32 * S::BN; e += S::THREADS) {
    const int64_t m = m0 + e / S::BN, n = n0 + e % S::BN;
    if (m >= G.M || n >= G.N) continue;
    const int64_t nk = G.Kp / 32;
    float acc = 0.0f;
    for (int64_t k = 0; k < G.Kp; ++k) {
      const __bf16* ar = G.ap + frag_index(m, k, nk);
      const __bf16* br = G.bp + frag_index(n, k, nk);
      const float a = (static_cast<float>(ar[0]) + static_cast<float>(ar[a_pl])) +
                      static_cast<float>(ar[2 * a_pl]);
      float b = static_cast<float>(br[0]);
      if (S::BP == 2) b += static_cast<float>(br[b_pl]);
      acc += a * b;
    }
    const float sc = G.scale ? load_as_f32(G.scale, G.scale_dt, n * G.scale_stride) : 1.0f;
    float v = acc * sc;
    if (G.alpha != 1.0f) v *= G.alpha;
    G.out[m * G.som + n * G.son] = v;
  }
}

// Runs f(integral_constant<U>, t + U) for U = 0 .. R - 1 while t + U < end.
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

template <class S>
__global__ void __launch_bounds__(S::THREADS) gemm_bf16_kernel(Args G) {
  constexpr int NT = S::NT, KS = S::KS, BP = S::BP, L = S::LOADS, R = S::RING;
  __shared__ float red[KS][NT][16][64];  // partial tiles, [wave][tile][register][lane]

  // the wave index as a uniform value, so that the K loop's bounds and
  // branches are scalar
  const int lane = threadIdx.x & 63,
            wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * 32;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * S::BN;
  const int64_t Kp = G.Kp;
  const int nk = static_cast<int>(Kp / 32);
  const int s0 = wave * nk / KS, s1 = (wave + 1) * nk / KS;  // this wave's K-steps
  if constexpr (BP == 2) {
    if (*G.flag == G.seq) {  // a non-finite operand in this call
      exact_tile<S>(G);
      return;
    }
  }

  // this lane's chunk of K-step 0, half 0 of the block's row tile of A and
  // first column tile of B; K-step s, half h is 1024 s + 512 h further, the
  // next column tile 1024 nk further
  const __bf16* a_fr = G.ap + frag_chunk(m0 >> 5, 0, 0, lane, nk);
  const __bf16* b_fr = G.bp + frag_chunk(n0 >> 5, 0, 0, lane, nk);
  const int64_t a_pl = G.Mp * Kp, b_pl = G.Np * Kp, b_t = 1024 * static_cast<int64_t>(nk);

  u4 ring[R][L];  // [slot][A plane x half, then B (tile, plane) x half]
  auto fetch = [&](int sl, int s) {
    const int64_t k0 = static_cast<int64_t>(s) * 1024;
#pragma unroll
    for (int p = 0; p < 3; ++p)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        ring[sl][2 * p + h] = *reinterpret_cast<const u4*>(a_fr + p * a_pl + k0 + 512 * h);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int p = 0; p < BP; ++p)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          ring[sl][6 + 2 * (t * BP + p) + h] =
              *reinterpret_cast<const u4*>(b_fr + t * b_t + p * b_pl + k0 + 512 * h);
  };

  f16v acc[NT][2];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int g = 0; g < 16; ++g) acc[t][h][g] = 0.0f;

  auto multiply = [&](auto uc) {
    constexpr int u = decltype(uc)::value;
#pragma unroll
    for (int pa = 0; pa < 3; ++pa)
#pragma unroll
      for (int pb = 0; pb < BP; ++pb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            const bf8 a = __builtin_bit_cast(bf8, ring[u][2 * pa + h]);
            const bf8 b = __builtin_bit_cast(bf8, ring[u][6 + 2 * (t * BP + pb) + h]);
            acc[t][h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[t][h], 0, 0, 0);
          }
  };
  // step s multiplies ring slot (s - s0) % R and refills it with step s + R:
  // always (step), while there is one (step_tail), or not at all (step_last).
  // The barrier keeps each refill in its step: scheduled later it would
  // leave the next round's first step waiting on a fresh burst of loads.
  auto step = [&](auto uc, int s) {
    multiply(uc);
    fetch(decltype(uc)::value, s + R);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto step_tail = [&](auto uc, int s) {
    multiply(uc);
    if (s + R < s1) fetch(decltype(uc)::value, s + R);  // (s and s1 are uniform)
    __builtin_amdgcn_sched_barrier(0);
  };
  auto step_last = [&](auto uc, int) { multiply(uc); };
  if (s1 - s0 >= R) {
#pragma unroll
    for (int u = 0; u < R; ++u) fetch(u, s0 + u);
    // whole rounds of R steps whose refills all exist (straight-line bodies,
    // so the loads in flight are the same at every round's start and each
    // step waits only for its own slot); then the round that refills what
    // is left (fewer than 2R steps remain), then the rest
    int t = s0;
    for (; t + 2 * R <= s1; t += R) Unroll<0, R>::run(step, t, t + R);
    Unroll<0, R>::run(step_tail, t, t + R);
    Unroll<0, R>::run(step_last, t + R, s1);
  } else if (s0 < s1) {  // fewer steps than ring slots
#pragma unroll
    for (int u = 0; u < R; ++u)
      if (s0 + u < s1) fetch(u, s0 + u);
    Unroll<0, R>::run(step_last, s0, s1);
  }

  // every wave's partial tile to LDS; wave w then sums registers
  // w * SHARE .. + SHARE - 1 (over the tiles) in wave order
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < 16; ++g) red[wave][t][g][lane] = acc[t][0][g] + acc[t][1][g];
  __syncthreads();

  float sc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int64_t n = n0 + 32 * t + (lane & 31);
    sc[t] = G.scale && n < G.N ? load_as_f32(G.scale, G.scale_dt, n * G.scale_stride) : 1.0f;
  }
  const float alpha = G.alpha;
  // D(i, j) of a 32x32 tile: lane j + 32 * ((i / 4) % 2), register (i / 8) * 4 + i % 4
#pragma unroll
  for (int i = 0; i < S::SHARE; ++i) {
    const int e = wave * S::SHARE + i, t = e / 16, g = e % 16;
    float v = red[0][t][g][lane];
#pragma unroll
    for (int w = 1; w < KS; ++w) v += red[w][t][g][lane];
    const int64_t n = n0 + 32 * t + (lane & 31);
    const int64_t m = m0 + 8 * (g / 4) + 4 * (lane >> 5) + (g % 4);
    if (m >= G.M || n >= G.N) continue;
    v *= sc[t];
    if (alpha != 1.0f) v *= alpha;
    G.out[m * G.som + n * G.son] = v;
  }
}

}  // namespace gdq

// Runs out = A @ dequant(B) on the bf16 matrix cores when the operands fit
// (see the top of the file); returns false, launching nothing, otherwise:
// A fp32 with K contiguous (K % 4 == 0, 16-byte aligned rows), B int8/uint8
// (scale, zero point of the same type or none) or fp16 (no dequantisation)
// with N contiguous and N % 4 == 0; batch axes only where B is shared and A
// and out are whole [batch * M] row ranges; the prepared operands within
// the scratch.
bool gemm_dq_try(const float* a, int64_t a_si, const void* b, int b_dt, int64_t b_si,
                 const Dequant& dq, float* out, int64_t som, int64_t son, const BatchMap& bm,
                 int64_t M, int64_t N, int64_t K, int64_t batch, float alpha, const int* only_if,
                 int* status) {
  using namespace gdq;
  *status = KK_OK;
  if (only_if) return false;
  const bool f16 = b_dt == KK_F16;
  if (f16) {
    if (dq.active || (reinterpret_cast<uintptr_t>(b) & 7)) return false;
  } else {
    if (!(b_dt == KK_I8 || b_dt == KK_U8)) return false;
    if (!dq.active || !dq.scale || (dq.zp && dq.zp_dt != b_dt)) return false;
    if (reinterpret_cast<uintptr_t>(b) & 3) return false;
  }
  if (K % 4 || a_si % 4 || (reinterpret_cast<uintptr_t>(a) & 15)) return false;
  if (N % 4 || b_si % 4) return false;
  // batch axes: B shared; A and out rows of consecutive batches follow on
  int64_t ea = M * a_si, eo = M * som;
  for (int d = bm.nb - 1; d >= 0; --d) {
    if (bm.dims[d] == 1) continue;
    if (bm.st[1][d] != 0 || bm.st[0][d] != ea || bm.st[2][d] != eo) return false;
    ea *= bm.dims[d];
    eo *= bm.dims[d];
  }
  const int bplanes = f16 ? 2 : 1;
  const int64_t Mt = M * batch;  // A and out as [batch * M] rows
  const int64_t Mp = ceil_div(Mt, kPadM) * kPadM, Np = ceil_div(N, kPadN) * kPadN,
                Kp = ceil_div(K, kPadK) * kPadK;
  const size_t a_bytes = static_cast<size_t>(3 * Mp * Kp) * 2;
  const size_t b_bytes = static_cast<size_t>(bplanes * Np * Kp) * 2;
  if (a_bytes + b_bytes > kScratchBytes || ceil_div(Mt, 32) > 65535 ||
      ceil_div(N, 32) > (int64_t{1} << 30))
    return false;

  char* scratch = static_cast<char*>(ctx().scratch);
  PrepArgs pa{a, a_si, b, b_si, b_dt, f16 ? nullptr : dq.zp, dq.zp_stride,
              reinterpret_cast<__bf16*>(scratch), reinterpret_cast<__bf16*>(scratch + a_bytes),
              Mt, N, K, Mp, Np, Kp, 0, nullptr, 0};
  int* flag = ctx().row_counters + kRowCounters + kFlagGemmBf16;
  int seq = 0;
  if (f16) {
    seq = ctx().gemm_seq = ctx().gemm_seq == 0x7fffffff ? 1 : ctx().gemm_seq + 1;
    pa.flag = flag;
    pa.seq = seq;
  }
  pa.a_blocks = static_cast<int>(ceil_div(Mp * Kp / 8, 256));
  const int64_t b_blocks = (Kp / 64) * (Np / 64);
  hipLaunchKernelGGL(gemm_dq_prep, dim3(static_cast<unsigned>(pa.a_blocks + b_blocks)), dim3(256), 0,
                     ctx().stream, pa);
  *status = check_launch("gemm_dq_prep");
  if (*status != KK_OK) return true;

  const Args g{pa.ap, pa.bp, f16 ? nullptr : dq.scale, dq.scale_dt, dq.scale_stride, out, som,
               son, Mt, N, Mp, Np, Kp, alpha, flag, seq};
  // 32 x 64 tiles when they cover every CU (eight waves for 8-bit weights,
  // four for fp16, whose ring of fourteen loads a step leaves no registers
  // for a second wave per SIMD), else 32 x 32 tiles of four waves, else
  // 32 x 32 tiles of eight (more loads in flight per CU when the tiles are
  // few).  Measured at 256 x 768 x 2048: 7.2 us (eight waves) vs 7.6 (four).
  const int64_t cus = ctx().num_cus > 0 ? ctx().num_cus : 256;
  const int64_t mt = ceil_div(Mt, 32);
#ifdef KK_GDQ_SHAPE
  const int shape = KK_GDQ_SHAPE;  // a fixed tile shape (for measuring them one by one)
#else
  const int shape = mt * ceil_div(N, 64) >= cus ? 0 : mt * ceil_div(N, 32) >= cus ? 1 : 2;
#endif
#define KK_DQ_LAUNCH(SH)                                                                        \
  hipLaunchKernelGGL((gemm_bf16_kernel<SH>),                                                    \
                     dim3(static_cast<unsigned>(ceil_div(N, SH::BN)), static_cast<unsigned>(mt)), \
                     dim3(SH::THREADS), 0, ctx().stream, g)
#define KK_DQ_SHAPES(BPL)                \
  do {                                   \
    using SA = Shape<2, 4, BPL>;         \
    using SB = Shape<1, 4, BPL>;         \
    using SC = Shape<1, 8, BPL>;         \
    using SD = Shape<2, 8, BPL>;         \
    if (shape == 0 && BPL == 1) KK_DQ_LAUNCH(SD); \
    else if (shape == 0) KK_DQ_LAUNCH(SA); \
    else if (shape == 1) KK_DQ_LAUNCH(SB); \
    else if (shape == 2) KK_DQ_LAUNCH(SC); \
    else KK_DQ_LAUNCH(SD);               \
  } while (0)
  if (f16) KK_DQ_SHAPES(2);
  else KK_DQ_SHAPES(1);
#undef KK_DQ_SHAPES
#undef KK_DQ_LAUNCH
  *status = check_launch("gemm_bf16_kernel");
  return true;
}

}  // namespace kk
