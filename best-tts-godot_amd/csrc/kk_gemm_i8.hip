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
#include <type_traits>

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

}  // namespace i8gemm
using namespace i8gemm;

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

}  // namespace kk

using namespace kk;

extern "C" {

int kk_matmul_integer(const kk_tensor* out, const kk_tensor* a, const kk_tensor* b,
                      const kk_tensor* a_zp, const kk_tensor* b_zp) {
  I8Args G;
  int64_t batch = 0;
  KK_TRY(i8_setup(&G, &batch, out, a, b, a_zp, b_zp, KK_I32, "kk_matmul_integer"));
  if (G.M == 0 || G.N == 0 || batch == 0) return KK_OK;
  if (G.K == 0) return kk_fill(out, 0.0);
  return i8_launch(G, batch);
}

int kk_matmul_integer_scaled(const kk_tensor* out, const kk_tensor* a, const kk_tensor* b,
                             const kk_tensor* a_zp, const kk_tensor* b_zp, const kk_tensor* scale,
                             const kk_tensor* scale2, const kk_tensor* bias) {
  const char* who = "kk_matmul_integer_scaled";
  I8Args G;
  int64_t batch = 0;
  KK_TRY(i8_setup(&G, &batch, out, a, b, a_zp, b_zp, KK_F32, who));
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
  return i8_launch(G, batch);
}

}  // extern "C"
