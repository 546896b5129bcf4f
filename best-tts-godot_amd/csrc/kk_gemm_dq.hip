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
// first: the same value up to fp32 rounding.
//
// One launch.  A block owns a 32 x (32 NT) output tile; each of its KS
// waves takes a run of 32-wide K-steps and, per step, loads the raw
// operands with coalesced 16-byte buffer loads (A: 32 rows x 128 bytes of
// fp32; B: 32 k rows of 32 NT weights) into a register ring that keeps the
// next steps in flight, stages them in its own LDS region (no block
// barrier in the K loop), reads them back as matrix-core operands -- A rows
// with 16-byte reads, B columns with the transposing reads
// ds_read_b64_tr_b8 (8-bit: each lane gets 8 consecutive k of its column)
// or ds_read_b64_tr_b16 (fp16: 4 consecutive k per read) -- splits and
// converts them in registers and accumulates into 2 NT independent 32x32
// tiles (one per half of each K-step).  The waves' partial tiles are summed
// through LDS in wave order.  Buffer loads past an operand's last byte
// return zeros, so rows past M, weight rows past K and the ragged edges
// need no per-lane branches; activation columns past K (the next row's
// values when K is not a multiple of 32) are cleared in the last K-step.
// Non-finite operands need no check per value: split without a guard, an
// infinite activation gives a1 = inf - inf = NaN (likewise b1 for an
// infinite fp16 weight, and a NaN gives NaN parts), and a NaN part makes
// every output it meets NaN on the matrix cores (NaN * 0 is NaN), so a
// block whose accumulators hold a NaN computes its tile with scalar fp32
// products instead (numpy's inf / NaN pattern).  Any other NaN there
// (overflowing sums) takes that path too, which is exact as well.
//
// What was measured on the way (per call at 256 x 768 x 2048 int8 / fp16
// 256 x 768 x 768): operands prepared by a first launch (A as three bf16
// planes, B converted and transposed, in the matrix-core fragment order)
// and a GEMM loading them straight into registers, 12.3 / 11.7 us -- two
// dependent launches, each waiting on a full memory round trip, and 6
// bytes of activation planes per value through L2; this one launch,
// 8.7 / 6.9 us.  A check per value for non-finite operands compiled to
// about 3.5 VALU instructions a value (the loop is VALU-bound) and gave way
// to the accumulator test.
#include <algorithm>
#include <mutex>
#include <type_traits>
#include <unordered_map>

#include "kk_internal.h"

namespace kk {
// Bytes of a [K, N] weight packed by kk_gemm_pack: per 32-column tile, per
// 32-wide K-step, per half-step, one 1 KB matrix-core fragment per bf16
// part (8-bit weights: q - z, one part; fp16: two parts).
int64_t gemm_packed_size(int64_t K, int64_t N, int w_dt) {
  return ceil_div(N, 32) * ceil_div(K, 32) * 2 * (w_dt == KK_F16 ? 2 : 1) * 1024;
}

namespace gfu {

// The upper halves of lo and hi as two packed bf16 (lo first).
__device__ __forceinline__ unsigned pack_hi(unsigned lo, unsigned hi) {
  return __builtin_amdgcn_perm(hi, lo, 0x07060302u);
}


typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));
typedef int i2v __attribute__((ext_vector_type(2)));
typedef short s4v __attribute__((ext_vector_type(4)));
#define KK_LDS __attribute__((address_space(3)))

// NT 32-wide column tiles, KS waves splitting K, BT bytes per weight (1:
// 8-bit, 2: fp16).  Staging pitches keep the LDS reads free of bank
// conflicts: A rows of 144 bytes (16 rows of a 16-byte read land on
// distinct banks), B rows of 32 / 96 bytes (8-bit, two 16-lane groups of
// transposing reads over 8 rows cover the 64 banks once) or 64 bytes (fp16,
// 4 rows).
template <int NT_, int KS_, int BT_, bool PB_ = false>
struct Shape {
  static constexpr int NT = NT_, KS = KS_, BT = BT_;
  // PB: B packed by kk_gemm_pack, read straight into registers as
  // matrix-core operands (PARTS bf16 fragments a tile and half-step)
  static constexpr bool PB = PB_;
  static constexpr int PARTS = BT;
  static constexpr int BN = 32 * NT, THREADS = 64 * KS;
  static constexpr int A_PITCH = 144;
  static constexpr int B_ROW = BN * BT;  // bytes of one k row of the B tile
  static constexpr int B_PITCH = BT == 1 ? (NT == 2 ? 96 : 32) : 64;
  static constexpr int B_CH = B_ROW / 16;          // 16-byte chunks per B row
  static constexpr int B_LOADS = 32 * B_CH / 64;   // 16-byte B loads per lane per K-step
  static constexpr int LOADS = 4 + (PB ? NT * 2 * PARTS : B_LOADS);
  static constexpr int STAGE = 32 * A_PITCH + (PB ? 0 : 32 * B_PITCH);  // one wave's staging bytes
  static constexpr int RED = KS * NT * 16 * 64 * 4;          // the partial tiles
  // PB: the partial tiles beside the staging (no barrier before they are
  // written); else in the staging's place
  static constexpr int RED_OFF = PB ? KS * STAGE : 0;
  static constexpr int LDS = PB ? KS * STAGE + RED : (KS * STAGE > RED ? KS * STAGE : RED);
  static constexpr int RING = KS == 8 ? 2 : 3;  // (two waves per SIMD share the registers)
  static constexpr int SHARE = NT * 16 / KS;
  static constexpr int B_ROWS_PER_LOAD = 64 / B_CH;  // B rows one 16-byte load per lane covers
  static_assert(BT == 1 || NT == 1, "fp16 weights: 32-wide column tiles");
  static_assert(B_LOADS * 64 == 32 * B_CH && SHARE * KS == NT * 16, "staging shape");
};

struct Args {
  const float* a;     // [Mt, K], rows a_si apart
  const void* b;      // [K, N], rows b_si apart (elements)
  uint32_t a_bytes, b_bytes;  // extents from each base (past them loads return zeros)
  int64_t a_si, b_si;
  int b_dt;
  const void* zp;     // 8-bit zero point or NULL
  int64_t zp_stride;
  const void* scale;  // per tensor or per column, or NULL (1)
  int scale_dt;
  int64_t scale_stride;
  float* out;
  int64_t som, son;
  int64_t M, N, K;
  float alpha;
  const void* bp;     // B packed by kk_gemm_pack (PB kernels)
  uint32_t bp_bytes;
};

__device__ __forceinline__ float zero_point(const Args& G, int64_t n) {
  if (!G.zp || n >= G.N) return 0.0f;
  const uint8_t zb = static_cast<const uint8_t*>(G.zp)[n * G.zp_stride];
  return G.b_dt == KK_I8 ? static_cast<float>(static_cast<int8_t>(zb)) : static_cast<float>(zb);
}

// The tile with scalar fp32 products of the raw operands, summed in k order.
template <class S>
__device__ void exact_tile(const Args& G, int64_t m0, int64_t n0) {
  for (int e = threadIdx.x; e < 32 * S::BN; e += S::THREADS) {
    const int64_t m = m0 + e / S::BN, n = n0 + e % S::BN;
    if (m >= G.M || n >= G.N) continue;
    const float* ar = G.a + m * G.a_si;
    float acc = 0.0f;
    if (S::BT == 2) {
      const _Float16* bc = static_cast<const _Float16*>(G.b) + n;
      for (int64_t k = 0; k < G.K; ++k) acc += ar[k] * static_cast<float>(bc[k * G.b_si]);
    } else {
      const float z = zero_point(G, n);
      const bool i8 = G.b_dt == KK_I8;
      const uint8_t* bc = static_cast<const uint8_t*>(G.b) + n;
      for (int64_t k = 0; k < G.K; ++k) {
        const uint8_t q = bc[k * G.b_si];
        const float qf = i8 ? static_cast<float>(static_cast<int8_t>(q)) : static_cast<float>(q);
        acc += ar[k] * (qf - z);
      }
    }
    const float sc = G.scale ? load_as_f32(G.scale, G.scale_dt, n * G.scale_stride) : 1.0f;
    float v = acc * sc;
    if (G.alpha != 1.0f) v *= G.alpha;
    G.out[m * G.som + n * G.son] = v;
  }
}

template <class S>
__global__ void __launch_bounds__(S::THREADS) gemm_fused_kernel(Args G) {
  constexpr int NT = S::NT, KS = S::KS, BT = S::BT, L = S::LOADS, R = S::RING;
  __shared__ __align__(16) unsigned char lds[S::LDS];
  __shared__ int bad_w[KS];

  const int lane = threadIdx.x & 63,
            wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * 32;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * S::BN;
  const int nk = static_cast<int>((G.K + 31) / 32);
  const int s0 = wave * nk / KS, s1 = (wave + 1) * nk / KS;  // this wave's K-steps

  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(G.a), 0, static_cast<int>(G.a_bytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(G.b), 0, static_cast<int>(G.b_bytes), 0x00020000);
  // this lane's loads: A row lane / 8 + 8 i, 16 bytes at 16 (lane % 8) of
  // the K-step's 128; B row lane / B_CH + B_ROWS_PER_LOAD i, chunk
  // lane % B_CH.  The whole offset goes in the per-lane register (the
  // range check that returns zeros past the extent covers that offset), the
  // row group's and K-step's parts formed as scalars.
  const int a_off = static_cast<int>((m0 + (lane >> 3)) * G.a_si * 4 + 16 * (lane & 7));
  const int a_st = (lane >> 3) * S::A_PITCH + 16 * (lane & 7);
  const int b_off = static_cast<int>((lane / S::B_CH) * G.b_si * BT + n0 * BT + 16 * (lane % S::B_CH));
  const int b_st = 32 * S::A_PITCH + (lane / S::B_CH) * S::B_PITCH + 16 * (lane % S::B_CH);
  const int a_grp = static_cast<int>(8 * G.a_si * 4), a_step = 128;
  const int b_grp = static_cast<int>(S::B_ROWS_PER_LOAD * G.b_si * BT),
            b_step = static_cast<int>(32 * G.b_si * BT);

  unsigned char* st = lds + wave * S::STAGE;
  u4 ring[R][L];
  // packed B: fragment ((tile * nk + s) * 2 + h) * PARTS + part, 1 KB each,
  // lane l's 16 bytes at 16 l
  const __amdgpu_buffer_rsrc_t rbp =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(G.bp), 0, static_cast<int>(G.bp_bytes), 0x00020000);
  const int bp_off = static_cast<int>((n0 / 32) * nk * 2 * S::PARTS * 1024 + 16 * lane);
  auto fetch = [&](int sl, int s) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ring[sl][i] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off + (s * a_step + i * a_grp), 0, 0);
    if constexpr (S::PB) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int pt = 0; pt < S::PARTS; ++pt)
            ring[sl][4 + (t * 2 + h) * S::PARTS + pt] = __builtin_amdgcn_raw_buffer_load_b128(
                rbp, bp_off + ((((t * nk + s) * 2 + h) * S::PARTS + pt) * 1024), 0, 0);
    } else {
#pragma unroll
      for (int i = 0; i < S::B_LOADS; ++i)
        ring[sl][4 + i] =
            __builtin_amdgcn_raw_buffer_load_b128(rb, b_off + (s * b_step + i * b_grp), 0, 0);
    }
  };

  // per-lane constants of the operand reads and conversions
  const int g = lane >> 5, r16 = lane & 15, grp = (lane >> 4) & 1;
  const int a_rd = (lane & 31) * S::A_PITCH + 64 * g;  // + 32 h: 8 fp32 of row lane % 32
  int b_rd[NT][2][2];  // [tile][half][read]: transposing-read addresses within the B region
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        if (BT == 1)  // 8 rows x 16 bytes per group: lane r gives row r / 2, bytes 8 (r % 2)
          b_rd[t][h][e] = (16 * g + 8 * h + (r16 >> 1)) * S::B_PITCH + 32 * t + 16 * grp +
                          8 * (r16 & 1);
        else  // 4 rows x 16 halves per group and read: lane r gives row r / 4, halves 4 (r % 4)
          b_rd[t][h][e] = (16 * g + 8 * h + 4 * e + (r16 >> 2)) * S::B_PITCH + 32 * grp +
                          8 * (r16 & 3);
      }
  const unsigned xmask = G.b_dt == KK_I8 ? 0x80808080u : 0u;  // int8 bytes as uint8 + 128
  float zoff[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
    zoff[t] = zero_point(G, n0 + 32 * t + (lane & 31)) + (G.b_dt == KK_I8 ? 128.0f : 0.0f);

  f16v acc[NT][2];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[t][h][q] = 0.0f;
  auto multiply = [&](auto uc, int s) {
    constexpr int u = decltype(uc)::value;
    // stage this step's raw operands in the wave's region
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u4*>(st + a_st + 8 * S::A_PITCH * i) = ring[u][i];
    if constexpr (!S::PB) {
#pragma unroll
      for (int i = 0; i < S::B_LOADS; ++i)
        *reinterpret_cast<u4*>(st + b_st + S::B_ROWS_PER_LOAD * S::B_PITCH * i) = ring[u][4 + i];
    }
    // read them back as operands
    float av[2][8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float4 x0 = *reinterpret_cast<const float4*>(st + a_rd + 32 * h);
      const float4 x1 = *reinterpret_cast<const float4*>(st + a_rd + 32 * h + 16);
      av[h][0] = x0.x; av[h][1] = x0.y; av[h][2] = x0.z; av[h][3] = x0.w;
      av[h][4] = x1.x; av[h][5] = x1.y; av[h][6] = x1.z; av[h][7] = x1.w;
    }
    unsigned bw[NT][2][4];  // raw weights: 8 bytes (8-bit) or 8 halves (fp16) per tile and half
    KK_LDS unsigned char* sb = (KK_LDS unsigned char*)(st) + 32 * S::A_PITCH;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if constexpr (S::PB) continue;
        if (BT == 1) {
          const i2v w = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
              reinterpret_cast<KK_LDS i2v*>(sb + b_rd[t][h][0]));
          bw[t][h][0] = w[0];
          bw[t][h][1] = w[1];
        } else {
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const s4v w = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                reinterpret_cast<KK_LDS s4v*>(sb + b_rd[t][h][e]));
            bw[t][h][2 * e] = static_cast<unsigned short>(w[0]) |
                              (static_cast<unsigned>(static_cast<unsigned short>(w[1])) << 16);
            bw[t][h][2 * e + 1] = static_cast<unsigned short>(w[2]) |
                                  (static_cast<unsigned>(static_cast<unsigned short>(w[3])) << 16);
          }
        }
      }
    // activation columns past K hold the next row's values: clear them
    if (s == nk - 1 && (G.K & 31)) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (32 * s + 16 * g + 8 * h + j >= G.K) av[h][j] = 0.0f;
    }
    // A: three bf16 parts per half
    bf8 ap[3][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      unsigned p0[4], p1[4], p2[4];
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        unsigned q0[2], q1[2], q2[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float x = av[h][j + e];
                    const unsigned ux = __float_as_uint(x);
          const float r = x - __uint_as_float(ux & 0xffff0000u);
          const unsigned ur = __float_as_uint(r);
          q0[e] = ux;
          q1[e] = ur;
          q2[e] = __float_as_uint(r - __uint_as_float(ur & 0xffff0000u));
        }
        p0[j / 2] = pack_hi(q0[0], q0[1]);
        p1[j / 2] = pack_hi(q1[0], q1[1]);
        p2[j / 2] = pack_hi(q2[0], q2[1]);
      }
      ap[0][h] = __builtin_bit_cast(bf8, u4{p0[0], p0[1], p0[2], p0[3]});
      ap[1][h] = __builtin_bit_cast(bf8, u4{p1[0], p1[1], p1[2], p1[3]});
      ap[2][h] = __builtin_bit_cast(bf8, u4{p2[0], p2[1], p2[2], p2[3]});
    }
    // B: bf16 operands (8-bit: q - z exact; fp16: two exact parts)
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if constexpr (S::PB) {
          const bf8 b0 = __builtin_bit_cast(bf8, ring[u][4 + (t * 2 + h) * S::PARTS]);
          if constexpr (BT == 1) {
#pragma unroll
            for (int pa = 0; pa < 3; ++pa)
              acc[t][h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[pa][h], b0, acc[t][h], 0, 0, 0);
          } else {
            const bf8 b1 = __builtin_bit_cast(bf8, ring[u][4 + (t * 2 + h) * S::PARTS + 1]);
#pragma unroll
            for (int pa = 0; pa < 3; ++pa) {
              acc[t][h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[pa][h], b0, acc[t][h], 0, 0, 0);
              acc[t][h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[pa][h], b1, acc[t][h], 0, 0, 0);
            }
          }
        } else if (BT == 1) {
          unsigned pb[4];
#pragma unroll
          for (int d = 0; d < 2; ++d) {
            const unsigned w = bw[t][h][d] ^ xmask;
            float f[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) f[c] = static_cast<float>((w >> (8 * c)) & 0xffu) - zoff[t];
            pb[2 * d] = pack_hi(__float_as_uint(f[0]), __float_as_uint(f[1]));
            pb[2 * d + 1] = pack_hi(__float_as_uint(f[2]), __float_as_uint(f[3]));
          }
          const bf8 b = __builtin_bit_cast(bf8, u4{pb[0], pb[1], pb[2], pb[3]});
#pragma unroll
          for (int pa = 0; pa < 3; ++pa)
            acc[t][h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[pa][h], b, acc[t][h], 0, 0, 0);
        } else {
          unsigned pb0[4], pb1[4];
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            unsigned q0[2], q1[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const float x = static_cast<float>(__builtin_bit_cast(
                  _Float16, static_cast<unsigned short>((bw[t][h][d] >> (16 * e)) & 0xffffu)));
                            const unsigned ux = __float_as_uint(x);
              q0[e] = ux;
              q1[e] = __float_as_uint(x - __uint_as_float(ux & 0xffff0000u));
            }
            pb0[d] = pack_hi(q0[0], q0[1]);
            pb1[d] = pack_hi(q1[0], q1[1]);
          }
          const bf8 b0 = __builtin_bit_cast(bf8, u4{pb0[0], pb0[1], pb0[2], pb0[3]});
          const bf8 b1 = __builtin_bit_cast(bf8, u4{pb1[0], pb1[1], pb1[2], pb1[3]});
#pragma unroll
          for (int pa = 0; pa < 3; ++pa) {
            acc[t][h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[pa][h], b0, acc[t][h], 0, 0, 0);
            acc[t][h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ap[pa][h], b1, acc[t][h], 0, 0, 0);
          }
        }
      }
  };
  // step s: stage and multiply ring slot (s - s0) % R, then refill it with
  // step s + R -- always (step), while there is one (step_tail), or not at
  // all (step_last).  The barrier keeps each refill in its step: scheduled
  // later, it left the next round's first step waiting on a fresh burst of
  // loads.
  auto step = [&](auto uc, int s) {
    multiply(uc, s);
    fetch(decltype(uc)::value, s + R);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto step_tail = [&](auto uc, int s) {
    multiply(uc, s);
    if (s + R < s1) fetch(decltype(uc)::value, s + R);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto step_last = [&](auto uc, int s) { multiply(uc, s); };
  if (s1 - s0 >= R) {
#pragma unroll
    for (int u = 0; u < R; ++u) fetch(u, s0 + u);
    int t = s0;
    // whole rounds of R steps whose refills all exist (straight-line bodies,
    // so the loads in flight are the same at every round's start and each
    // step waits only for its own slot); then the round that refills what
    // is left (fewer than 2R steps remain), then the rest
    for (; t + 2 * R <= s1; t += R) Unroll<0, R>::run(step, t, t + R);
    Unroll<0, R>::run(step_tail, t, t + R);
    Unroll<0, R>::run(step_last, t + R, s1);
  } else if (s0 < s1) {
#pragma unroll
    for (int u = 0; u < R; ++u)
      if (s0 + u < s1) fetch(u, s0 + u);
    Unroll<0, R>::run(step_last, s0, s1);
  }

  if constexpr (S::PB) {
    float sc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int64_t n = n0 + 32 * t + (lane & 31);
      sc[t] = G.scale && n < G.N ? load_as_f32(G.scale, G.scale_dt, n * G.scale_stride) : 1.0f;
    }
    // the partial tiles, summed in wave order; a NaN in any partial makes
    // its sum NaN, so the test runs on the sums (four a lane) rather than
    // on the accumulators (64 a lane)
    float* red = reinterpret_cast<float*>(lds + S::RED_OFF);  // [wave][tile][register][lane]
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int q = 0; q < 16; ++q) red[((wave * NT + t) * 16 + q) * 64 + lane] = acc[t][0][q] + acc[t][1][q];
    __syncthreads();
    float v[S::SHARE];
    bool vbad = false;
#pragma unroll
    for (int i = 0; i < S::SHARE; ++i) {
      const int e = wave * S::SHARE + i, t = e / 16, q = e % 16;
      v[i] = red[(t * 16 + q) * 64 + lane];
#pragma unroll
      for (int w = 1; w < KS; ++w) v[i] += red[((w * NT + t) * 16 + q) * 64 + lane];
      vbad |= __builtin_isnan(v[i]);
    }
    const int vwave_bad = __any(vbad);  // (all lanes active: the vote covers the whole wave)
    if (lane == 0) bad_w[wave] = vwave_bad;
    __syncthreads();
    bool vany_bad = false;
#pragma unroll
    for (int w = 0; w < KS; ++w) vany_bad |= bad_w[w] != 0;
    if (vany_bad) {
      exact_tile<S>(G, m0, n0);
      return;
    }
    // D(i, j) of a 32x32 tile: lane j + 32 * ((i / 4) % 2), register (i / 8) * 4 + i % 4
#pragma unroll
    for (int i = 0; i < S::SHARE; ++i) {
      const int e = wave * S::SHARE + i, t = e / 16, q = e % 16;
      const int64_t n = n0 + 32 * t + (lane & 31);
      const int64_t m = m0 + 8 * (q / 4) + 4 * (lane >> 5) + (q % 4);
      if (m >= G.M || n >= G.N) continue;
      float o = v[i] * sc[t];
      if (G.alpha != 1.0f) o *= G.alpha;
      G.out[m * G.som + n * G.son] = o;
    }
    return;
  }
  bool bad = false;  // a NaN in this lane's accumulators (see the top of the section)
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int q = 0; q < 16; ++q) bad |= __builtin_isnan(acc[t][h][q]);
  const int wave_bad = __any(bad);  // (all lanes active: the vote covers the whole wave)
  if (lane == 0) bad_w[wave] = wave_bad;
  __syncthreads();  // every wave is done with its staging (the partial tiles reuse it)
  bool any_bad = false;
#pragma unroll
  for (int w = 0; w < KS; ++w) any_bad |= bad_w[w] != 0;
  if (any_bad) {
    exact_tile<S>(G, m0, n0);
    return;
  }
  float* red = reinterpret_cast<float*>(lds);  // [wave][tile][register][lane]
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int q = 0; q < 16; ++q) red[((wave * NT + t) * 16 + q) * 64 + lane] = acc[t][0][q] + acc[t][1][q];
  __syncthreads();

  float sc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int64_t n = n0 + 32 * t + (lane & 31);
    sc[t] = G.scale && n < G.N ? load_as_f32(G.scale, G.scale_dt, n * G.scale_stride) : 1.0f;
  }
  // D(i, j) of a 32x32 tile: lane j + 32 * ((i / 4) % 2), register (i / 8) * 4 + i % 4
#pragma unroll
  for (int i = 0; i < S::SHARE; ++i) {
    const int e = wave * S::SHARE + i, t = e / 16, q = e % 16;
    float v = red[(t * 16 + q) * 64 + lane];
#pragma unroll
    for (int w = 1; w < KS; ++w) v += red[((w * NT + t) * 16 + q) * 64 + lane];
    const int64_t n = n0 + 32 * t + (lane & 31);
    const int64_t m = m0 + 8 * (q / 4) + 4 * (lane >> 5) + (q % 4);
    if (m >= G.M || n >= G.N) continue;
    v *= sc[t];
    if (G.alpha != 1.0f) v *= G.alpha;
    G.out[m * G.som + n * G.son] = v;
  }
}

struct PackArgs {
  const void* w;     // [K, N], rows w_si apart
  int w_dt;
  int64_t w_si;
  const void* zp;    // 8-bit zero point (per tensor or per column) or NULL
  int64_t zp_stride;
  int64_t K, N;
  int nk, parts;
  int64_t total;     // 16-byte units
  u4* out;
};

// One lane of one fragment per thread: fragment ((tile * nk + s) * 2 + h) *
// parts + part, lane l = (n, g) = (l % 32, l / 32) holding the weights of
// column 32 tile + n at k = 32 s + 16 g + 8 h + e, e = 0..7 -- the k order the
// kernel's staged activations take -- as bf16: q - z for 8-bit weights
// (exact), the two parts b0 + b1 of an fp16 weight.
__global__ void __launch_bounds__(256) gemm_pack_kernel(PackArgs P) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (u >= P.total) return;
  const int lane = static_cast<int>(u % 64);
  int64_t r = u / 64;
  const int pt = static_cast<int>(r % P.parts);
  r /= P.parts;
  const int h = static_cast<int>(r % 2);
  r /= 2;
  const int s = static_cast<int>(r % P.nk);
  const int64_t tile = r / P.nk;
  const int64_t n = 32 * tile + (lane & 31);
  const int g = lane >> 5;
  unsigned f[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t k = 32 * static_cast<int64_t>(s) + 16 * g + 8 * h + e;
    float v = 0.0f;
    if (k < P.K && n < P.N) {
      if (P.w_dt == KK_F16) {
        const float x = static_cast<float>(static_cast<const _Float16*>(P.w)[k * P.w_si + n]);
        const float x0 = __uint_as_float(__float_as_uint(x) & 0xffff0000u);
        v = pt == 0 ? x0 : x - x0;
      } else {
        const uint8_t qb = static_cast<const uint8_t*>(P.w)[k * P.w_si + n];
        const uint8_t zb = P.zp ? static_cast<const uint8_t*>(P.zp)[n * P.zp_stride] : 0;
        v = P.w_dt == KK_I8 ? static_cast<float>(static_cast<int8_t>(qb)) - static_cast<float>(static_cast<int8_t>(zb))
                            : static_cast<float>(qb) - static_cast<float>(zb);
      }
    }
    f[e] = __float_as_uint(v);
  }
  P.out[u] = u4{pack_hi(f[0], f[1]), pack_hi(f[2], f[3]), pack_hi(f[4], f[5]), pack_hi(f[6], f[7])};
}

// What a packed buffer was made from (checked by every packed call).
struct PackRecord {
  const void* w;
  int64_t K, N;
  int w_dt;
  const void* zp;
  int zp_dt;
};
static std::mutex g_pack_mu;
static std::unordered_map<const void*, PackRecord> g_packs;

}  // namespace gfu

void gemm_forget_pack(const void* p) {
  std::lock_guard<std::mutex> lock(gfu::g_pack_mu);
  gfu::g_packs.erase(p);
}

// Checks a packed buffer against a call's [K, N] weight w and zero point:
// its size and alignment, and that the last kk_gemm_pack into it read this
// very w and zero point.
int gemm_check_packed(const kk_tensor* packed, const kk_tensor* w, const kk_tensor* w_zp,
                      const char* who) {
  KK_TRY(check_tensor(packed, "packed"));
  if (w->rank != 2) return set_error(KK_E_ARG, "%s: a packed weight is [K, N]", who);
  const int64_t need = gemm_packed_size(w->shape[0], w->shape[1], w->dtype);
  if (packed->dtype != KK_U8 || !is_contiguous(packed) || numel(packed) != need ||
      reinterpret_cast<uintptr_t>(packed->data) % 256 != 0)
    return set_error(KK_E_ARG, "%s: packed must be %lld contiguous, 256-byte aligned uint8 bytes",
                     who, (long long)need);
  std::lock_guard<std::mutex> lock(gfu::g_pack_mu);
  auto it = gfu::g_packs.find(packed->data);
  if (it == gfu::g_packs.end()) return set_error(KK_E_ARG, "%s: packed was not made by kk_gemm_pack", who);
  const gfu::PackRecord& r = it->second;
  if (r.w != w->data || r.K != w->shape[0] || r.N != w->shape[1] || r.w_dt != w->dtype)
    return set_error(KK_E_ARG, "%s: packed was made from another weight tensor", who);
  if (r.zp != (w_zp ? w_zp->data : nullptr) || r.zp_dt != (w_zp ? w_zp->dtype : -1))
    return set_error(KK_E_ARG, "%s: packed was made with another weight zero point", who);
  return KK_OK;
}

// Launches the kernel when B's rows are 16-byte aligned and every offset a
// load forms is below 2^31; false, launching nothing, otherwise.
static bool gemm_fused_try(const float* a, int64_t a_si, const void* b, int b_dt, int64_t b_si,
                           const Dequant& dq, float* out, int64_t som, int64_t son, int64_t Mt,
                           int64_t N, int64_t K, float alpha, const void* bpack, int* status) {
  using namespace gfu;
  const int bt = b_dt == KK_F16 ? 2 : 1;
  if ((reinterpret_cast<uintptr_t>(b) & 15) || (b_si * bt) % 16) return false;
  const int64_t a_bytes = ((Mt - 1) * a_si + K) * 4, b_bytes = ((K - 1) * b_si + N) * bt;
  // the largest offset a load forms: a whole 32-row, 32-wide K-step past the extents
  const int64_t a_reach = (ceil_div(Mt, 32) * 32 * a_si + ceil_div(K, 32) * 32) * 4;
  const int64_t b_reach = (ceil_div(K, 32) * 32 * b_si + ceil_div(N, 64) * 64) * bt;
  if (a_reach >= (int64_t{1} << 31) || b_reach >= (int64_t{1} << 31)) return false;
  const int64_t bp_bytes = gemm_packed_size(K, N, b_dt);
  if (bpack && bp_bytes >= (int64_t{1} << 31)) return false;
  const Args g{a, b, static_cast<uint32_t>(a_bytes), static_cast<uint32_t>(b_bytes), a_si, b_si,
               b_dt, bt == 1 ? dq.zp : nullptr, dq.zp_stride, bt == 1 ? dq.scale : nullptr,
               dq.scale_dt, dq.scale_stride, out, som, son, Mt, N, K, alpha, bpack,
               static_cast<uint32_t>(bpack ? bp_bytes : 0)};
  const int64_t cus = ctx().num_cus > 0 ? ctx().num_cus : 256;
  const int64_t mt = ceil_div(Mt, 32);
#ifdef KK_GFU_SHAPE
  const int shape = KK_GFU_SHAPE;  // a fixed tile shape (for measuring them one by one)
#else
  const int shape = bt == 1 && mt * ceil_div(N, 64) >= cus ? 0 : 1;
#endif
#define KK_GFU_LAUNCH(SH)                                                                       \
  KK_LAUNCH((gemm_fused_kernel<SH>),                                                   \
                     dim3(static_cast<unsigned>(ceil_div(N, SH::BN)), static_cast<unsigned>(mt)), \
                     dim3(SH::THREADS), 0, ctx().stream, g)
  using H4 = Shape<1, 4, 2>;
  using H8 = Shape<1, 8, 2>;
  using Q64x8 = Shape<2, 8, 1>;
  using Q32x8 = Shape<1, 8, 1>;
  using Q32x4 = Shape<1, 4, 1>;
  using Q64x4 = Shape<2, 4, 1>;
  using PH8 = Shape<1, 8, 2, true>;
  using PQ64x8 = Shape<2, 8, 1, true>;
  using PQ32x8 = Shape<1, 8, 1, true>;
  if (bpack) {
    if (bt == 2) KK_GFU_LAUNCH(PH8);
    else if (shape == 0) KK_GFU_LAUNCH(PQ64x8);
    else KK_GFU_LAUNCH(PQ32x8);
  } else if (bt == 2) {
    if (shape == 2) KK_GFU_LAUNCH(H4);
    else KK_GFU_LAUNCH(H8);
  } else {
    if (shape == 0) KK_GFU_LAUNCH(Q64x8);
    else if (shape == 2) KK_GFU_LAUNCH(Q32x4);
    else if (shape == 3) KK_GFU_LAUNCH(Q64x4);
    else KK_GFU_LAUNCH(Q32x8);
  }
#undef KK_GFU_LAUNCH
  *status = check_launch("gemm_fused_kernel");
  return true;
}


// Runs out = A @ dequant(B) on the bf16 matrix cores when the operands fit
// (see the top of the file); returns false, launching nothing, otherwise:
// A fp32 with K contiguous (K % 4 == 0, 16-byte aligned rows), B int8/uint8
// (scale, zero point of the same type or none) or fp16 (no dequantisation)
// with N contiguous and 16-byte aligned rows; batch axes only where B is
// shared and A and out are whole [batch * M] row ranges.
bool gemm_dq_try(const float* a, int64_t a_si, const void* b, int b_dt, int64_t b_si,
                 const Dequant& dq, float* out, int64_t som, int64_t son, const BatchMap& bm,
                 int64_t M, int64_t N, int64_t K, int64_t batch, float alpha, const int* only_if,
                 const void* bpack, int* status) {
  *status = KK_OK;
  if (only_if) return false;
  if (b_dt == KK_F16) {
    if (dq.active) return false;
  } else {
    if (!(b_dt == KK_I8 || b_dt == KK_U8)) return false;
    if (!dq.active || !dq.scale || (dq.zp && dq.zp_dt != b_dt)) return false;
  }
  if (K % 4 || a_si % 4 || (reinterpret_cast<uintptr_t>(a) & 15)) return false;
  // batch axes: B shared; A and out rows of consecutive batches follow on
  int64_t ea = M * a_si, eo = M * som;
  for (int d = bm.nb - 1; d >= 0; --d) {
    if (bm.dims[d] == 1) continue;
    if (bm.st[1][d] != 0 || bm.st[0][d] != ea || bm.st[2][d] != eo) return false;
    ea *= bm.dims[d];
    eo *= bm.dims[d];
  }
  const int64_t Mt = M * batch;  // A and out as [batch * M] rows
  if (ceil_div(Mt, 32) > 65535 || ceil_div(N, 32) > (int64_t{1} << 30)) return false;
  return gemm_fused_try(a, a_si, b, b_dt, b_si, dq, out, som, son, Mt, N, K, alpha, bpack, status);
}

}  // namespace kk

using namespace kk;

extern "C" {

int kk_gemm_packed_bytes(int64_t k, int64_t n, int w_dtype, int64_t* bytes) {
  if (!bytes || k <= 0 || n <= 0)
    return set_error(KK_E_ARG, "kk_gemm_packed_bytes: positive sizes and an output");
  if (!(w_dtype == KK_F16 || w_dtype == KK_I8 || w_dtype == KK_U8))
    return set_error(KK_E_ARG, "kk_gemm_packed_bytes: int8, uint8 or fp16 weights");
  *bytes = gemm_packed_size(k, n, w_dtype);
  return KK_OK;
}

int kk_gemm_pack(const kk_tensor* packed, const kk_tensor* w, const kk_tensor* w_zp) {
  const char* who = "kk_gemm_pack";
  KK_TRY(require_ready());
  KK_TRY(check_tensor(w, "w"));
  if (w->rank != 2 || !(w->dtype == KK_F16 || w->dtype == KK_I8 || w->dtype == KK_U8) ||
      w->strides[1] != 1 || numel(w) == 0)
    return set_error(KK_E_ARG, "%s: w must be a non-empty fp16/int8/uint8 [K, N] with N contiguous",
                     who);
  const int64_t K = w->shape[0], N = w->shape[1];
  int64_t zp_stride = 0;
  if (w_zp) {
    if (w->dtype == KK_F16) return set_error(KK_E_ARG, "%s: an fp16 weight takes no zero point", who);
    KK_TRY(check_tensor(w_zp, "w_zp"));
    if (w_zp->dtype != w->dtype)
      return set_error(KK_E_ARG, "%s: w_zp must have w's type", who);
    const int64_t nz = numel(w_zp);
    if (nz == N && nz > 1) {
      zp_stride = w_zp->rank ? w_zp->strides[w_zp->rank - 1] : 0;
    } else if (nz != 1) {
      return set_error(KK_E_ARG, "%s: w_zp must be per tensor or per column", who);
    }
  }
  const int64_t bytes = gemm_packed_size(K, N, w->dtype);
  if (bytes >= (int64_t{1} << 31))
    return set_error(KK_E_UNSUPPORTED, "%s: %lld packed bytes exceed 2 GiB", who, (long long)bytes);
  KK_TRY(check_tensor(packed, "packed"));
  if (packed->dtype != KK_U8 || !is_contiguous(packed) || numel(packed) != bytes ||
      reinterpret_cast<uintptr_t>(packed->data) % 256 != 0)
    return set_error(KK_E_ARG, "%s: packed must be %lld contiguous, 256-byte aligned uint8 bytes",
                     who, (long long)bytes);
  {
    std::lock_guard<std::mutex> lock(gfu::g_pack_mu);
    gfu::g_packs[packed->data] =
        gfu::PackRecord{w->data, K, N, w->dtype, w_zp ? w_zp->data : nullptr, w_zp ? w_zp->dtype : -1};
  }
  gfu::PackArgs P{w->data, w->dtype, w->strides[0], w_zp ? w_zp->data : nullptr, zp_stride, K, N,
                  static_cast<int>(ceil_div(K, 32)), w->dtype == KK_F16 ? 2 : 1, bytes / 16,
                  static_cast<gfu::u4*>(packed->data)};
  KK_LAUNCH(gfu::gemm_pack_kernel, dim3(static_cast<unsigned>(ceil_div(P.total, 256))), dim3(256), 0,
            ctx().stream, P);
  return check_launch("gemm_pack_kernel");
}

}  // extern "C"
