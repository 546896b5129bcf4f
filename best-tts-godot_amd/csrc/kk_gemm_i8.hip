// MatMulInteger on the int8 matrix cores (v_mfma_i32_32x32x32_i8), exact in
// int32: op_matmul_integer (ref_runtime.py:119-127) computes
// int32 (a - a_zp) @ (b - b_zp); its GLSL twin kernels/matmul_int8.glsl:55-62
// accumulates in int as well.
//
// Both operands are offset into int8 (a uint8 byte u becomes u - 128 =
// u ^ 0x80; an int8 byte stays as it is), and so are the zero points, so
//   sum_k (a'_k - az')(b'_k - bz') = sum_k a'_k b'_k - bz' sum_k a'_k
//                                    - az' sum_k b'_k + K az' bz'
// The first sum runs on the MFMA; the row sums of a' and the column sums of
// b' come from the tiles staged in LDS (v_dot4 with ones).  Every term is
// int32 arithmetic, exact modulo 2^32, so the result is the exact integer
// result modulo 2^32 -- what numpy's int32 matmul gives, and the exact value
// whenever it fits int32 (always for K <= 33025: |a - az|, |b - bz| <= 255).
//
// Block: 64 x 64 outputs, 4 waves as 2 x 2, each a 32 x 32 MFMA tile; K-steps
// of 256 (the graph's K of 768 and 2048 in 3 and 8 steps: at its M of 130
// a launch has a few dozen blocks, each waiting out one round trip a step).
// A [M, K] is staged row-major (K contiguous, 16-byte loads); B
// [K, N] arrives N-contiguous and is transposed on the way into LDS (a
// thread loads four rows of four columns, one dword each, and swaps the 4 x 4
// bytes with v_perm), so both MFMA operand fragments -- 16 consecutive k of
// one row or column -- are single 16-byte LDS reads.  The next K-step is
// loaded into registers while this one is multiplied.  The fused
// Cast -> Mul(scale) (-> Add(bias)) tail of the graph runs in the epilogue.
#include <mutex>
#include <type_traits>
#include <unordered_map>

#include "kk_internal.h"

namespace kk {
namespace i8gemm {  // named: the kernels keep readable names in profiles

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kTM = 64, kTN = 64;  // outputs per block
constexpr int kTK = 256;           // K-step (bytes of one row)
constexpr int kPitch = kTK + 16;   // LDS row pitch: 16-byte pad staggers the banks
constexpr int kThreads = 256;
constexpr int kAPieces = kTM * kTK / 16 / kThreads;         // 16-byte A pieces a thread
constexpr int kBItems = (kTK / 4) * (kTN / 4) / kThreads;   // 4 x 4-byte B items a thread
constexpr int kRowPieces = kTK / 16;

struct I8Args {
  const uint8_t* a;     // bytes of A [.., M, K]
  int64_t a_si, a_sj;
  uint32_t a_flip;      // 0x80808080 for uint8 A, else 0
  const uint8_t* b;     // bytes of B [.., K, N]
  int64_t b_si, b_sj;
  uint32_t b_flip;
  const void* azp;      // one value or NULL
  int azp_dt;
  const void* bzp;      // 1 or N values or NULL
  int bzp_dt;
  int64_t bzp_stride;   // 0 (per tensor) or 1 (per column)
  BatchMap bm;
  int64_t M, N, K;
  int32_t* out_i;       // int32 result, or NULL when out_f is set
  float* out_f;         // float(result) * (cs[n] * cs2[n]) (+ cb[n])
  int64_t som, son;
  const float* cs;
  int64_t cs_n;
  const float* cs2;
  int64_t cs2_n;
  const float* cb;
  int64_t cb_n;
  // packed B (i8_packed_kernel): fragments, column sums of b', k-steps
  const uint8_t* bp;
  const int32_t* colsum;
  int nS;
};

// AV: A rows 16-byte loadable (K % 16 == 0, aligned); BV: B rows dword
// loadable (N % 4 == 0, aligned).  Otherwise byte gathers.
template <bool AV, bool BV>
__global__ void __launch_bounds__(kThreads) i8_matmul_kernel(I8Args G) {
  __shared__ __align__(16) int8_t As[2][kTM * kPitch];
  __shared__ __align__(16) int8_t Bs[2][kTN * kPitch];
  __shared__ int sums[kTM + kTN];  // row sums of a', then column sums of b'
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int r = lane & 31, g = lane >> 5;
  const int wm = wv >> 1, wn = wv & 1;
  const uint3 tile = xcd_tile();  // neighbouring column tiles on one XCD
  const int64_t bz = tile.z;
  const int64_t m0 = static_cast<int64_t>(tile.y) * kTM;
  const int64_t n0 = static_cast<int64_t>(tile.x) * kTN;
  const int64_t M = G.M, N = G.N, K = G.K;
  const uint8_t* a = G.a + batch_offset(G.bm, 0, bz);
  const uint8_t* b = G.b + batch_offset(G.bm, 1, bz);
  // The vector paths read through buffer resources based at this block's
  // first row of A and first column of B (the host keeps each span below
  // 2^31 bytes).  An offset at or past the span reads zeros, so the bounds
  // become a select on the offset: a guarded load would be a branch with a
  // wait of its own, and the K-step's loads would go out one at a time.
  const int64_t a_rows = M - m0 < kTM ? M - m0 : kTM;
  const uint32_t a_span = static_cast<uint32_t>((a_rows - 1) * G.a_si + K);
  const uint32_t b_span = static_cast<uint32_t>((K - 1) * G.b_si + (N - n0));
  const auto a_rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a + m0 * G.a_si), 0,
                                                      static_cast<int>(a_span), 0x00020000);
  const auto b_rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(b + n0), 0,
                                                      static_cast<int>(b_span), 0x00020000);

  // A pieces: kAPieces a thread, row i / kRowPieces, 16 bytes at k 16 (i % kRowPieces)
  v4i ra[kAPieces];
  uint32_t fa[kAPieces] = {};  // the flip of a vector piece, applied as it is stashed
  auto fetch_a = [&](int64_t k0) {
#pragma unroll
    for (int j = 0; j < kAPieces; ++j) {
      const int i = tid + kThreads * j, row = i / kRowPieces, kc = 16 * (i % kRowPieces);
      const int64_t m = m0 + row, k = k0 + kc;
      v4i v = {0, 0, 0, 0};  // padding holds a' = 0
      if (AV) {
        const bool in = m < M && k < K;
        const uint32_t off = in ? static_cast<uint32_t>(row * G.a_si + k) : a_span;
        v = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(a_rs, off, 0, 0));
        fa[j] = in ? G.a_flip : 0u;
      } else {
        uint32_t w[4] = {0, 0, 0, 0};
        if (m < M) {
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (k + e < K)
              w[e >> 2] |= (static_cast<uint32_t>(a[m * G.a_si + (k + e) * G.a_sj]) ^ (G.a_flip & 0xffu))
                           << (8 * (e & 3));
        }
        v = v4i{static_cast<int>(w[0]), static_cast<int>(w[1]), static_cast<int>(w[2]),
                static_cast<int>(w[3])};
      }
      ra[j] = v;
    }
  };
  auto stash_a = [&](int buf) {
#pragma unroll
    for (int j = 0; j < kAPieces; ++j) {
      const int i = tid + kThreads * j;
      *reinterpret_cast<v4i*>(&As[buf][(i / kRowPieces) * kPitch + 16 * (i % kRowPieces)]) =
          ra[j] ^ static_cast<int>(fa[j]);
    }
  };
  // B items: kBItems a thread, rows k 4 (i >> 4) .. +3 x columns 4 (i & 15) .. +3
  uint32_t rb[kBItems][4];
  uint32_t fb[kBItems][4] = {};  // as fa
  auto fetch_b = [&](int64_t k0) {
#pragma unroll
    for (int j = 0; j < kBItems; ++j) {
      const int i = tid + kThreads * j, kg = i >> 4, ng = i & 15;
      const int64_t n = n0 + 4 * ng;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t k = k0 + 4 * kg + q;
        uint32_t v = 0;  // padding holds b' = 0
        if (BV) {
          const bool in = k < K && n < N;
          const uint32_t off = in ? static_cast<uint32_t>(k * G.b_si + 4 * ng) : b_span;
          v = __builtin_amdgcn_raw_buffer_load_b32(b_rs, off, 0, 0);
          fb[j][q] = in ? G.b_flip : 0u;
        } else if (k < K) {
          {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n + e < N)
                v |= (static_cast<uint32_t>(b[k * G.b_si + (n + e) * G.b_sj]) ^ (G.b_flip & 0xffu))
                     << (8 * e);
          }
        }
        rb[j][q] = v;
      }
    }
  };
  auto stash_b = [&](int buf) {
#pragma unroll
    for (int j = 0; j < kBItems; ++j) {
      const int i = tid + kThreads * j, kg = i >> 4, ng = i & 15;
      uint32_t d[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) d[q] = rb[j][q] ^ fb[j][q];
      // 4 x 4 byte transpose (v_perm: bytes 0-3 from the second operand, 4-7
      // from the first): word e = column 4ng + e at rows 4kg .. 4kg + 3
      const uint32_t t01l = __builtin_amdgcn_perm(d[1], d[0], 0x05010400u);
      const uint32_t t01h = __builtin_amdgcn_perm(d[1], d[0], 0x07030602u);
      const uint32_t t23l = __builtin_amdgcn_perm(d[3], d[2], 0x05010400u);
      const uint32_t t23h = __builtin_amdgcn_perm(d[3], d[2], 0x07030602u);
      int8_t* dst = &Bs[buf][(4 * ng) * kPitch + 4 * kg];
      *reinterpret_cast<uint32_t*>(dst) = __builtin_amdgcn_perm(t23l, t01l, 0x05040100u);
      *reinterpret_cast<uint32_t*>(dst + kPitch) = __builtin_amdgcn_perm(t23l, t01l, 0x07060302u);
      *reinterpret_cast<uint32_t*>(dst + 2 * kPitch) = __builtin_amdgcn_perm(t23h, t01h, 0x05040100u);
      *reinterpret_cast<uint32_t*>(dst + 3 * kPitch) = __builtin_amdgcn_perm(t23h, t01h, 0x07060302u);
    }
  };

  // row / column sums: thread t sums half (t & 1) of staged row t >> 1
  // (rows 0-63 of As, then 0-63 of Bs); the even lane keeps the total
  const int srow = tid >> 1, shalf = tid & 1;
  int my_sum = 0;
  const int a_off = (wm * 32 + r) * kPitch + 16 * g;
  const int b_off = (wn * 32 + r) * kPitch + 16 * g;
  v16i acc = {};
  const int64_t nk = ceil_div(K, kTK);
  fetch_a(0);
  fetch_b(0);
  stash_a(0);
  stash_b(0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int buf = static_cast<int>(kt & 1);
    const bool more = kt + 1 < nk;
    if (more) {
      fetch_a((kt + 1) * kTK);
      fetch_b((kt + 1) * kTK);
    }
#pragma unroll
    for (int ks = 0; ks < kTK / 32; ++ks) {
      const v4i af = *reinterpret_cast<const v4i*>(&As[buf][a_off + 32 * ks]);
      const v4i bf = *reinterpret_cast<const v4i*>(&Bs[buf][b_off + 32 * ks]);
      acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf, acc, 0, 0, 0);
    }
    {
      const int8_t* src = (srow < kTM ? &As[buf][srow * kPitch] : &Bs[buf][(srow - kTM) * kPitch]) +
                          (kTK / 2) * shalf;
      int s = 0;
#pragma unroll
      for (int q = 0; q < kTK / 8; ++q)
        s = __builtin_amdgcn_sdot4(reinterpret_cast<const int*>(src)[q], 0x01010101, s, false);
      s += __shfl_xor(s, 1, 64);
      my_sum += s;
    }
    if (more) {
      stash_a(buf ^ 1);
      stash_b(buf ^ 1);
    }
    __syncthreads();
  }
  if (shalf == 0) sums[srow] = my_sum;
  __syncthreads();

  // v = acc - bz' sum a' - az' sum b' + K az' bz'  (int32, modulo 2^32)
  const int azo = (G.azp ? static_cast<int>(load_as_i64(G.azp, G.azp_dt, 0)) : 0) -
                  (G.a_flip ? 128 : 0);
  const int jl = wn * 32 + r;  // this lane's column in the tile
  const int64_t n = n0 + jl;
  if (n >= N) return;
  const int bzo = (G.bzp ? static_cast<int>(load_as_i64(G.bzp, G.bzp_dt, n * G.bzp_stride)) : 0) -
                  (G.b_flip ? 128 : 0);
  // unsigned: wrap-around arithmetic, modulo 2^32
  const uint32_t uaz = static_cast<uint32_t>(azo), ubz = static_cast<uint32_t>(bzo);
  const uint32_t colterm = static_cast<uint32_t>(K) * uaz * ubz -
                           uaz * static_cast<uint32_t>(sums[kTM + jl]);
  float sc = 0.0f, bias = 0.0f;
  if (G.out_f) {
    sc = G.cs[G.cs_n > 1 ? n : 0];
    if (G.cs2) sc = sc * G.cs2[G.cs2_n > 1 ? n : 0];
    if (G.cb) bias = G.cb[G.cb_n > 1 ? n : 0];
  }
  const int64_t oo = batch_offset(G.bm, 2, bz);
  // D(i, j) of the 32 x 32 tile: lane j + 32 ((i / 4) % 2), register
  // (i / 8) 4 + i % 4
#pragma unroll
  for (int reg = 0; reg < 16; ++reg) {
    const int il = wm * 32 + 8 * (reg / 4) + 4 * g + (reg % 4);
    const int64_t m = m0 + il;
    if (m >= M) continue;
    const int v = static_cast<int>(static_cast<uint32_t>(acc[reg]) -
                                   ubz * static_cast<uint32_t>(sums[il]) + colterm);
    const int64_t o = oo + m * G.som + n * G.son;
    if (G.out_f) {
      float y = static_cast<float>(v) * sc;
      if (G.cb) y = y + bias;
      G.out_f[o] = y;
    } else {
      G.out_i[o] = v;
    }
  }
}

// ------------------------------------------------------- packed weights
// kk_matmul_integer_pack lays a constant [K, N] B out as the MFMA takes it:
// for column tile t (32 columns) and k-step s (32 k), 64 lanes x 16 bytes,
// lane (n, g) holding b'[32 s + 16 g + e][32 t + n] for e = 0..15 (zeros past
// K and N; b' = b for int8, b - 128 for uint8), tiles t-major so that one
// tile's k-steps are contiguous; then the N column sums of b' (int32,
// modulo 2^32).  A wave loads a fragment with one 16-byte load a lane,
// straight into registers: no LDS stage, no transpose, and the column sums
// are not recomputed per call.
inline int64_t pack_frag_bytes(int64_t K, int64_t N) {
  return ceil_div(N, 32) * ceil_div(K, 32) * 1024;
}

__global__ void __launch_bounds__(256) i8_pack_kernel(uint4* __restrict__ dst,
                                                      const uint8_t* __restrict__ b, int64_t b_si,
                                                      int64_t b_sj, int64_t K, int64_t N, int nS,
                                                      uint32_t flip, int64_t pieces) {
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < pieces;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int lane = static_cast<int>(idx % 64);
    const int64_t ts = idx / 64, st = ts % nS, t = ts / nS;
    const int64_t n = 32 * t + (lane & 31), k0 = 32 * st + 16 * (lane >> 5);
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    if (n < N) {
      for (int e = 0; e < 16; ++e)
        if (k0 + e < K)
          w[e >> 2] |= ((static_cast<uint32_t>(b[(k0 + e) * b_si + n * b_sj]) ^ flip) & 0xffu)
                       << (8 * (e & 3));
    }
    dst[idx] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

__global__ void __launch_bounds__(256) i8_colsum_kernel(int32_t* __restrict__ cs,
                                                        const uint8_t* __restrict__ b, int64_t b_si,
                                                        int64_t b_sj, int64_t K, int64_t N,
                                                        uint32_t flip) {
  const int64_t n = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (n >= N) return;
  uint32_t sum = 0;
  for (int64_t k = 0; k < K; ++k)
    sum += static_cast<uint32_t>(static_cast<int32_t>(
        static_cast<int8_t>((static_cast<uint32_t>(b[k * b_si + n * b_sj]) ^ flip) & 0xffu)));
  cs[n] = static_cast<int32_t>(sum);
}

// MatMulInteger on packed B, one 32 x 32 output tile a block: the four
// waves split the k-steps, each loading its share of A (one 16-byte piece a
// lane: row lane % 32, k 16 (lane / 32) of the step, out of range reading
// zeros) and of the packed B, SPW steps in flight before it multiplies, and
// summing its rows of a' on the side (v_dot4 with ones); waves 1-3 hand
// their accumulators and row sums to wave 0 through LDS, which corrects for
// the zero points as i8_matmul_kernel does and runs the epilogue.  A and
// the output are contiguous, their batch dimensions folded into the rows
// (B is one [K, N] matrix).
template <int SPW>
__global__ void __launch_bounds__(kThreads) i8_packed_kernel(I8Args G) {
  __shared__ int red[3][16][64];
  __shared__ int rsum[4][32];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int r = lane & 31, g = lane >> 5;
  const int64_t t = blockIdx.x, m0 = static_cast<int64_t>(blockIdx.y) * 32;
  const int64_t M = G.M, N = G.N, K = G.K;
  const int nS = G.nS;
  const int64_t a_rows = M - m0 < 32 ? M - m0 : 32;
  const uint32_t a_span = static_cast<uint32_t>((a_rows - 1) * G.a_si + K);
  const auto a_rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(G.a + m0 * G.a_si), 0,
                                                      static_cast<int>(a_span), 0x00020000);
  const uint32_t b_span = static_cast<uint32_t>(nS) * 1024u;
  const auto b_rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(G.bp + t * static_cast<int64_t>(nS) * 1024), 0, static_cast<int>(b_span),
      0x00020000);
  const int per = (nS + 3) / 4;
  const int s0 = w * per, s1 = s0 + per < nS ? s0 + per : nS;
  const bool row_in = r < a_rows;
  v16i acc = {};
  int rs = 0;
  const uint32_t a_row = static_cast<uint32_t>(r * G.a_si) + 16u * g;
  const uint32_t kg = 16u * g;
  const uint32_t K32 = static_cast<uint32_t>(K);
  for (int c = s0; c < s1; c += SPW) {
    v4i av[SPW], bv[SPW];
#pragma unroll
    for (int u = 0; u < SPW; ++u) {
      const int st = c + u;
      const bool in = st < s1 && row_in && 32u * st + kg < K32;
      av[u] = __builtin_bit_cast(
          v4i, __builtin_amdgcn_raw_buffer_load_b128(a_rs, in ? a_row + 32u * st : a_span, 0, 0));
      bv[u] = __builtin_bit_cast(
          v4i, __builtin_amdgcn_raw_buffer_load_b128(
                   b_rs, st < s1 ? static_cast<uint32_t>(st * 64 + lane) * 16u : b_span, 0, 0));
    }
#pragma unroll
    for (int u = 0; u < SPW; ++u) {
      const int st = c + u;
      const bool in = st < s1 && row_in && 32u * st + kg < K32;
      const v4i a2 = av[u] ^ static_cast<int>(in ? G.a_flip : 0u);
      acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a2, bv[u], acc, 0, 0, 0);
#pragma unroll
      for (int q = 0; q < 4; ++q) rs = __builtin_amdgcn_sdot4(a2[q], 0x01010101, rs, false);
    }
  }
  rs += __shfl_xor(rs, 32, 64);  // the row's two k halves
  if (g == 0) rsum[w][r] = rs;
  if (w > 0) {
#pragma unroll
    for (int reg = 0; reg < 16; ++reg) red[w - 1][reg][lane] = acc[reg];
  }
  __syncthreads();
  if (w > 0) return;
#pragma unroll
  for (int reg = 0; reg < 16; ++reg)
    acc[reg] = static_cast<int>(static_cast<uint32_t>(acc[reg]) +
                                static_cast<uint32_t>(red[0][reg][lane]) +
                                static_cast<uint32_t>(red[1][reg][lane]) +
                                static_cast<uint32_t>(red[2][reg][lane]));
  const int64_t n = 32 * t + r;  // this lane's column
  if (n >= N) return;
  const int azo = (G.azp ? static_cast<int>(load_as_i64(G.azp, G.azp_dt, 0)) : 0) -
                  (G.a_flip ? 128 : 0);
  const int bzo = (G.bzp ? static_cast<int>(load_as_i64(G.bzp, G.bzp_dt, n * G.bzp_stride)) : 0) -
                  (G.b_flip ? 128 : 0);
  const uint32_t uaz = static_cast<uint32_t>(azo), ubz = static_cast<uint32_t>(bzo);
  const uint32_t colterm = static_cast<uint32_t>(K) * uaz * ubz -
                           uaz * static_cast<uint32_t>(G.colsum[n]);
  float sc = 0.0f, bias = 0.0f;
  if (G.out_f) {
    sc = G.cs[G.cs_n > 1 ? n : 0];
    if (G.cs2) sc = sc * G.cs2[G.cs2_n > 1 ? n : 0];
    if (G.cb) bias = G.cb[G.cb_n > 1 ? n : 0];
  }
#pragma unroll
  for (int reg = 0; reg < 16; ++reg) {
    const int il = 8 * (reg / 4) + 4 * g + (reg % 4);
    if (il >= a_rows) continue;
    const uint32_t rsm = static_cast<uint32_t>(rsum[0][il]) + static_cast<uint32_t>(rsum[1][il]) +
                         static_cast<uint32_t>(rsum[2][il]) + static_cast<uint32_t>(rsum[3][il]);
    const int v = static_cast<int>(static_cast<uint32_t>(acc[reg]) - ubz * rsm + colterm);
    const int64_t o = (m0 + il) * G.som + n;
    if (G.out_f) {
      float y = static_cast<float>(v) * sc;
      if (G.cb) y = y + bias;
      G.out_f[o] = y;
    } else {
      G.out_i[o] = v;
    }
  }
}

struct I8PackRecord {
  const void* b;
  int64_t K, N;
  int b_dt;
};
static std::mutex g_i8_pack_mu;
static std::unordered_map<const void*, I8PackRecord> g_i8_packs;

}  // namespace i8gemm
using namespace i8gemm;

void i8_forget_pack(const void* p) {
  std::lock_guard<std::mutex> lock(g_i8_pack_mu);
  g_i8_packs.erase(p);
}

static int64_t i8_packed_size(int64_t K, int64_t N) {
  return pack_frag_bytes(K, N) + ceil_div(4 * N, 256) * 256;
}

// Checks a packed buffer against a call's [K, N] B: size, alignment, and
// that the last kk_matmul_integer_pack into it read this very B.
static int i8_check_packed(const kk_tensor* packed, const kk_tensor* b, const char* who) {
  KK_TRY(check_tensor(packed, "packed"));
  if (b->rank != 2) return set_error(KK_E_ARG, "%s: a packed B is [K, N]", who);
  const int64_t need = i8_packed_size(b->shape[0], b->shape[1]);
  if (packed->dtype != KK_U8 || !is_contiguous(packed) || numel(packed) != need ||
      reinterpret_cast<uintptr_t>(packed->data) % 256 != 0)
    return set_error(KK_E_ARG, "%s: packed must be %lld contiguous, 256-byte aligned uint8 bytes",
                     who, (long long)need);
  std::lock_guard<std::mutex> lock(g_i8_pack_mu);
  auto it = g_i8_packs.find(packed->data);
  if (it == g_i8_packs.end())
    return set_error(KK_E_ARG, "%s: packed was not made by kk_matmul_integer_pack", who);
  const I8PackRecord& rec = it->second;
  if (rec.b != b->data || rec.K != b->shape[0] || rec.N != b->shape[1] || rec.b_dt != b->dtype)
    return set_error(KK_E_ARG, "%s: packed was made from another B", who);
  return KK_OK;
}

static bool aligned_to(const void* p, int bytes) {
  return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

// Shapes, dtypes and zero points of MatMulInteger (ref_runtime.py:119-127);
// `out_dt` is int32 (the plain op) or fp32 (the fused tail).
static int i8_setup(I8Args* G, int64_t* batch, const kk_tensor* out, const kk_tensor* a,
                    const kk_tensor* b, const kk_tensor* a_zp, const kk_tensor* b_zp, int out_dt,
                    const char* who) {
  *G = I8Args{};
  KK_TRY(matmul_shape(out, a, b, &G->bm, &G->M, &G->N, &G->K, batch, who));
  if (!(a->dtype == KK_U8 || a->dtype == KK_I8) || !(b->dtype == KK_U8 || b->dtype == KK_I8))
    return set_error(KK_E_ARG, "%s: a and b must be uint8/int8", who);
  if (out->dtype != out_dt)
    return set_error(KK_E_ARG, "%s: out must be %s", who, out_dt == KK_I32 ? "int32" : "fp32");
  Dequant az, bzq;
  KK_TRY(zp_shift(&az, a_zp, 1, who));
  KK_TRY(zp_shift(&bzq, b_zp, G->N, who));
  G->a = static_cast<const uint8_t*>(a->data);
  G->a_si = a->strides[a->rank - 2];
  G->a_sj = a->strides[a->rank - 1];
  G->a_flip = a->dtype == KK_U8 ? 0x80808080u : 0u;
  G->b = static_cast<const uint8_t*>(b->data);
  G->b_si = b->strides[b->rank - 2];
  G->b_sj = b->strides[b->rank - 1];
  G->b_flip = b->dtype == KK_U8 ? 0x80808080u : 0u;
  G->azp = az.zp;
  G->azp_dt = az.zp_dt;
  G->bzp = bzq.zp;
  G->bzp_dt = bzq.zp_dt;
  G->bzp_stride = bzq.zp_stride;
  G->som = out->strides[out->rank - 2];
  G->son = out->strides[out->rank - 1];
  if (out_dt == KK_I32) G->out_i = static_cast<int32_t*>(out->data);
  else G->out_f = static_cast<float*>(out->data);
  return KK_OK;
}

static int i8_launch(const I8Args& G, int64_t batch) {
  const int64_t gy = ceil_div(G.M, kTM), gx = ceil_div(G.N, kTN);
  if (gy > 65535 || batch > 65535 || gx > 0x7fffffff)
    return set_error(KK_E_UNSUPPORTED, "MatMulInteger: grid %lld x %lld x %lld too large",
                     (long long)gx, (long long)gy, (long long)batch);
  bool av = G.a_sj == 1 && G.K % 16 == 0 && G.a_si % 16 == 0 && aligned_to(G.a, 16);
  bool bv = G.b_sj == 1 && G.N % 4 == 0 && G.b_si % 4 == 0 && aligned_to(G.b, 4);
  for (int d = 0; d < G.bm.nb; ++d) {
    if (G.bm.st[0][d] % 16) av = false;
    if (G.bm.st[1][d] % 4) bv = false;
  }
  // the buffer spans of one block's rows of A and of B's K rows
  const int64_t kSpanMax = (int64_t{1} << 31) - 256;
  if ((std::min<int64_t>(G.M, kTM) - 1) * G.a_si + G.K > kSpanMax) av = false;
  if ((G.K - 1) * G.b_si + G.N > kSpanMax) bv = false;
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy), static_cast<unsigned>(batch));
  KK_TRY(check_xcd_grid(grid, "MatMulInteger"));
  hipStream_t st = ctx().stream;
  if (av && bv) KK_LAUNCH((i8_matmul_kernel<true, true>), grid, dim3(kThreads), 0, st, G);
  else if (av) KK_LAUNCH((i8_matmul_kernel<true, false>), grid, dim3(kThreads), 0, st, G);
  else if (bv) KK_LAUNCH((i8_matmul_kernel<false, true>), grid, dim3(kThreads), 0, st, G);
  else KK_LAUNCH((i8_matmul_kernel<false, false>), grid, dim3(kThreads), 0, st, G);
  return check_launch("i8_matmul_kernel");
}

// Launches i8_packed_kernel when A and the output are contiguous (their
// batch dimensions folded into the rows), A's rows are 16-byte loadable
// and every offset stays below 2^31; false, launching nothing, otherwise
// (the caller then runs i8_matmul_kernel on b itself).
static bool i8_packed_try(I8Args* G, const kk_tensor* out, const kk_tensor* a,
                          const kk_tensor* packed) {
  const int64_t K = G->K, N = G->N;
  if (!is_contiguous(a) || !is_contiguous(out) || K % 16 != 0 || !aligned_to(a->data, 16))
    return false;
  const int64_t rows = numel(a) / K;
  const int64_t nS = ceil_div(K, 32), gy = ceil_div(rows, 32), gx = ceil_div(N, 32);
  if (32 * K > (int64_t{1} << 31) - 256 || nS * 1024 > (int64_t{1} << 31) - 256 || gy > 65535 ||
      gx > 0x7fffffff)
    return false;
  G->M = rows;
  G->a_si = K;
  G->som = N;
  G->son = 1;
  G->bp = static_cast<const uint8_t*>(packed->data);
  G->colsum = reinterpret_cast<const int32_t*>(G->bp + pack_frag_bytes(K, N));
  G->nS = static_cast<int>(nS);
  const int per = static_cast<int>((nS + 3) / 4);
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  hipStream_t st = ctx().stream;
  if (per <= 1) KK_LAUNCH((i8_packed_kernel<1>), grid, dim3(kThreads), 0, st, *G);
  else if (per <= 2) KK_LAUNCH((i8_packed_kernel<2>), grid, dim3(kThreads), 0, st, *G);
  else if (per <= 4) KK_LAUNCH((i8_packed_kernel<4>), grid, dim3(kThreads), 0, st, *G);
  else if (per <= 6) KK_LAUNCH((i8_packed_kernel<6>), grid, dim3(kThreads), 0, st, *G);
  else if (per <= 8) KK_LAUNCH((i8_packed_kernel<8>), grid, dim3(kThreads), 0, st, *G);
  else if (per <= 12) KK_LAUNCH((i8_packed_kernel<12>), grid, dim3(kThreads), 0, st, *G);
  else KK_LAUNCH((i8_packed_kernel<16>), grid, dim3(kThreads), 0, st, *G);
  return true;
}

}  // namespace kk

using namespace kk;

extern "C" {

int kk_matmul_integer(const kk_tensor* out, const kk_tensor* a, const kk_tensor* b,
                      const kk_tensor* a_zp, const kk_tensor* b_zp) {
  return kk_matmul_integer_packed(out, a, b, nullptr, a_zp, b_zp);
}

int kk_matmul_integer_packed(const kk_tensor* out, const kk_tensor* a, const kk_tensor* b,
                             const kk_tensor* packed, const kk_tensor* a_zp,
                             const kk_tensor* b_zp) {
  const char* who = packed ? "kk_matmul_integer_packed" : "kk_matmul_integer";
  I8Args G;
  int64_t batch = 0;
  KK_TRY(i8_setup(&G, &batch, out, a, b, a_zp, b_zp, KK_I32, who));
  if (packed) KK_TRY(i8_check_packed(packed, b, who));
  if (G.M == 0 || G.N == 0 || batch == 0) return KK_OK;
  if (G.K == 0) return kk_fill(out, 0.0);
  if (packed && i8_packed_try(&G, out, a, packed)) return check_launch("i8_packed_kernel");
  return i8_launch(G, batch);
}

int kk_matmul_integer_scaled(const kk_tensor* out, const kk_tensor* a, const kk_tensor* b,
                             const kk_tensor* a_zp, const kk_tensor* b_zp, const kk_tensor* scale,
                             const kk_tensor* scale2, const kk_tensor* bias) {
  return kk_matmul_integer_scaled_packed(out, a, b, nullptr, a_zp, b_zp, scale, scale2, bias);
}

int kk_matmul_integer_scaled_packed(const kk_tensor* out, const kk_tensor* a, const kk_tensor* b,
                                    const kk_tensor* packed, const kk_tensor* a_zp,
                                    const kk_tensor* b_zp, const kk_tensor* scale,
                                    const kk_tensor* scale2, const kk_tensor* bias) {
  const char* who = packed ? "kk_matmul_integer_scaled_packed" : "kk_matmul_integer_scaled";
  I8Args G;
  int64_t batch = 0;
  KK_TRY(i8_setup(&G, &batch, out, a, b, a_zp, b_zp, KK_F32, who));
  if (packed) KK_TRY(i8_check_packed(packed, b, who));
  // scale and bias: one value or one per output column, contiguous fp32
  auto per_col = [&](const kk_tensor* t, const char* what, const float** p, int64_t* n) -> int {
    KK_TRY(check_tensor(t, what));
    if (t->dtype != KK_F32 || !is_contiguous(t))
      return set_error(KK_E_ARG, "%s: %s must be contiguous fp32", who, what);
    const int64_t c = numel(t);
    if (c != 1 && !(c == G.N && t->rank >= 1 && t->shape[t->rank - 1] == G.N))
      return set_error(KK_E_ARG, "%s: %s must hold 1 or N = %lld values", who, what,
                       (long long)G.N);
    *p = static_cast<const float*>(t->data);
    *n = c;
    return KK_OK;
  };
  if (!scale) return set_error(KK_E_ARG, "%s: scale is required", who);
  KK_TRY(per_col(scale, "scale", &G.cs, &G.cs_n));
  if (scale2) KK_TRY(per_col(scale2, "scale2", &G.cs2, &G.cs2_n));
  if (bias) KK_TRY(per_col(bias, "bias", &G.cb, &G.cb_n));
  if (G.M == 0 || G.N == 0 || batch == 0) return KK_OK;
  if (G.K == 0) return set_error(KK_E_UNSUPPORTED, "%s: K = 0", who);
  if (packed && i8_packed_try(&G, out, a, packed)) return check_launch("i8_packed_kernel");
  return i8_launch(G, batch);
}

int kk_matmul_integer_pack_bytes(const kk_tensor* b, size_t* bytes) {
  KK_TRY(check_tensor(b, "b"));
  if (!bytes) return set_error(KK_E_ARG, "kk_matmul_integer_pack_bytes: bytes is NULL");
  if (b->rank != 2 || !(b->dtype == KK_U8 || b->dtype == KK_I8) || b->shape[0] == 0 ||
      b->shape[1] == 0)
    return set_error(KK_E_ARG, "kk_matmul_integer_pack_bytes: b must be a non-empty [K, N] "
                               "int8/uint8 matrix");
  *bytes = static_cast<size_t>(i8_packed_size(b->shape[0], b->shape[1]));
  return KK_OK;
}

int kk_matmul_integer_pack(const kk_tensor* packed, const kk_tensor* b) {
  const char* who = "kk_matmul_integer_pack";
  KK_TRY(require_ready());
  size_t bytes = 0;
  KK_TRY(kk_matmul_integer_pack_bytes(b, &bytes));
  KK_TRY(check_tensor(packed, "packed"));
  if (packed->dtype != KK_U8 || !is_contiguous(packed) ||
      numel(packed) != static_cast<int64_t>(bytes) ||
      reinterpret_cast<uintptr_t>(packed->data) % 256 != 0)
    return set_error(KK_E_ARG, "%s: packed must be %zu contiguous, 256-byte aligned uint8 bytes",
                     who, bytes);
  const int64_t K = b->shape[0], N = b->shape[1];
  const int64_t nS = ceil_div(K, 32);
  if (nS > (int64_t{1} << 21))
    return set_error(KK_E_UNSUPPORTED, "%s: K = %lld too large", who, (long long)K);
  const uint32_t flip = b->dtype == KK_U8 ? 0x80u : 0u;
  const int64_t frag = pack_frag_bytes(K, N), pieces = frag / 16;
  uint8_t* dst = static_cast<uint8_t*>(packed->data);
  const uint8_t* src = static_cast<const uint8_t*>(b->data);
  hipStream_t st = ctx().stream;
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>(ceil_div(pieces, 256), 65536));
  KK_LAUNCH(i8_pack_kernel, dim3(grid), dim3(256), 0, st, reinterpret_cast<uint4*>(dst), src,
            b->strides[0], b->strides[1], K, N, static_cast<int>(nS), flip, pieces);
  KK_TRY(check_launch("i8_pack_kernel"));
  KK_LAUNCH(i8_colsum_kernel, dim3(static_cast<unsigned>(ceil_div(N, 256))), dim3(256), 0, st,
            reinterpret_cast<int32_t*>(dst + frag), src, b->strides[0], b->strides[1], K, N, flip);
  KK_TRY(check_launch("i8_colsum_kernel"));
  std::lock_guard<std::mutex> lock(g_i8_pack_mu);
  g_i8_packs[packed->data] = I8PackRecord{b->data, K, N, b->dtype};
  return KK_OK;
}

}  // extern "C"
