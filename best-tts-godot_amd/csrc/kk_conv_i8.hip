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
// Layout: the weights become CoutP x Kw x CinP bytes in MFMA fragment order
// (CinP = Cin rounded up to 64 with zero channels) with sum_k a_k per output
// channel, once per call.
// The activations stay as they are, uint8 [N][Cin][L]: each block stages
// the time window its outputs read, 64 channels at a time, into LDS
// time-major (channels contiguous, offset to int8 on the way), so each
// MFMA operand fragment -- 16 channels of one tap at one output row or time
// step -- is one 16-byte LDS read; the same staged rows give
// sum_ci b[t][ci] for the epilogue.
#include <type_traits>

#include <mutex>
#include <unordered_map>

#include "kk_internal.h"

namespace kk {
namespace i8conv {  // named: the kernels keep readable names in profiles

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kTileM = 128;  // output channels per block (2 waves x 64)
constexpr int kCinAlign = 64;   // channels per chunk: two 32-deep MFMA steps
constexpr int kRowPitch = 80;   // LDS bytes per 64-channel row (16-byte pad: staggered banks)
constexpr int kLeafPitch = 136; // LDS floats per output row in the leaf sums' transpose

// LDS of a block: the staged rows and their channel sums, the per-channel
// epilogue constants; with leaf sums, then the 64-row transpose area.
__host__ __device__ constexpr int conv_leaf_off(int rows) {
  return (rows * (kRowPitch + 4) + 2 * kTileM * 4 + 15) & ~15;
}
constexpr int kLeafBytes = 64 * kLeafPitch * 4;

// The graph's per-call bias quantisation ahead of a quantised conv:
// scale = Mul(sa, sw), bias_int32 = Cast(Floor(Div(bias, scale))); sa and sw
// one value each, bias Cout values.  qb.scale / qb.bias receive them.
struct QBias {
  const float* sa;
  const float* sw;
  const float* bias;
  float* scale;
  int32_t* ibias;
};

// The per-call bias quantisation of one channel: scale = sa * sw and
// int32 bias = Cast(Floor(Div(bias, scale))), each operation rounded as its
// node rounds it; the float -> int32 Cast as the device's Cast node does it
// (truncation, INT64_MIN outside the int64 range, then the low 32 bits).
__device__ inline int32_t qbias_channel(float sa, float sw, float b, float* scale) {
  const float sc = sa * sw;
  const float t = truncf(floorf(b / sc));
  const int64_t v = (t >= -9.223372036854775808e18f && t < 9.223372036854775808e18f)
                        ? static_cast<int64_t>(t) : INT64_MIN;
  *scale = sc;
  return static_cast<int32_t>(v);
}

// The offset weights (0 for padding rows/channels) in MFMA fragment order:
// for row block mb = co / 128, step st = (ci / 64) Kw + tap, wave row wm =
// (co % 128) / 64, fragment q = 2 ((ci % 64) / 32) + (co % 64) / 32 and lane
// l = co % 32 + 32 ((ci % 32) / 16), the 16 bytes ci % 16 = 0..15 sit at
// ((mb S + st) 2 + wm) 4096 + 1024 q + 16 l (S = Kw CinP / 64 steps);
// wsum[co] = sum of the offset weights; wzo[co] = offset weight zero point;
// with qb.scale set also channel co's quantised bias and scale.
__global__ void __launch_bounds__(256) conv_i8_wprep(const void* __restrict__ w, int w_dt,
                                                     const void* __restrict__ wzp, int wzp_dt,
                                                     int64_t wzp_n, int8_t* __restrict__ wT,
                                                     int32_t* __restrict__ wsum,
                                                     int32_t* __restrict__ wzo, int64_t Cout,
                                                     int64_t Cin, int64_t Kw, int64_t CinP,
                                                     QBias qb) {
  __shared__ int part[4];
  const int64_t co = blockIdx.x;
  const bool live = co < Cout;
  const int off = w_dt == KK_U8 ? 128 : 0;
  const int64_t S = Kw * (CinP / kCinAlign);
  const int rr = static_cast<int>(co % kTileM);
  const int64_t row_base = ((co / kTileM) * S * 2 + rr / 64) * 4096 + 1024 * ((rr / 32) % 2) +
                           16 * (rr % 32);
  int local = 0;
  for (int64_t idx = threadIdx.x; idx < Kw * (CinP / 16); idx += blockDim.x) {
    const int64_t tap = idx / (CinP / 16), ci0 = 16 * (idx % (CinP / 16));
    uint32_t wd[4];
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      uint32_t v = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t ci = ci0 + 4 * e4 + e;
        int a = 0;
        if (live && ci < Cin) {
          const int64_t src = (co * Cin + ci) * Kw + tap;
          a = w_dt == KK_U8 ? static_cast<int>(static_cast<const uint8_t*>(w)[src]) - 128
                            : static_cast<int>(static_cast<const int8_t*>(w)[src]);
        }
        local += a;
        v |= (static_cast<uint32_t>(a) & 0xffu) << (8 * e);
      }
      wd[e4] = v;
    }
    const int64_t st = (ci0 / kCinAlign) * Kw + tap, kk = ci0 % kCinAlign;
    const int64_t dst = row_base + st * 8192 + 2048 * (kk / 32) + 512 * ((kk / 16) % 2);
    *reinterpret_cast<uint4*>(wT + dst) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
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
    if (qb.scale && live) {
      float sc;
      qb.ibias[co] = qbias_channel(qb.sa[0], qb.sw[0], qb.bias[co], &sc);
      qb.scale[co] = sc;
    }
  }
}

struct ConvI8Args {
  const int8_t* wT;     // fragment order (conv_i8_wprep), CoutP Kw CinP bytes
  const int32_t* wsum;  // [CoutP]
  const int32_t* wzo;   // [CoutP] (live rows: the tensor's offset zero point)
  const uint8_t* x;     // [N][Cin][L]
  const uint8_t* xzp;   // one uint8 or NULL
  int32_t* out;         // [N][Cout][Lout] int32, or NULL when outf is set
  float* outf;          // [N][Cout][Lout] float(acc + bias[co]) * scale
  const int32_t* bias;  // [Cout] or NULL
  const float* scale;   // 1 or Cout values
  const float* resid;   // with outf: [N][Cout][Lout] added after the scale (the Add), or NULL
  const float* qsa;     // with outf, packed weights: scale = qsa[0] * qsw[0] and the int32
  const float* qsw;     // bias of channel co from the fp32 qbias[co] (qbias_channel), formed
  const float* qbias;   // in the prologue instead of the weight preparation
  int64_t scale_n;
  int64_t Cout, Cin, CinP, Kw, s, d, L, p0, Lout, Kreal;
  int W4;               // time rows staged per block: the window plus alignment slack
  int aligned;          // rows start 4-byte aligned (L % 4 == 0): dword loads
  // with outf and 128-step tiles: leaf[(n Cout + co) nleaf + t] = the sum of
  // the block's 128 outputs of row co at steps 128 t .. 128 t + 127 in
  // numpy's order, for t < nleaf (the leaves of the rows' whole 8192-blocks)
  float* leaf;
  int64_t nleaf;
};

// Block: 128 output channels x TN output steps, 4 waves as 2 (channels) x
// 2 (time), wave tile 64 x TN/2 as 2 x TN/64 MFMA tiles of 32 x 32.  For each
// 64-channel chunk the block stages its whole input window -- the
// ((TN - 1) s + (K - 1) d + 1) time rows every tap reads, each tap shifted by
// tap * d -- in LDS once, straight from the uint8 activations: a thread
// loads four time steps of four channels (one dword per channel), swaps the
// 4 x 4 bytes into four time rows and flips the top bit (u - 128 = u ^ 0x80);
// positions in the padding hold xz - 128.  The weights' MFMA fragments come
// from global memory in the order the waves read them (each wave's 4
// fragments of a (chunk, tap) step are 4 KB contiguous, loaded three steps
// ahead), so the taps run without LDS weight tiles or barriers.  Lane (r, g)
// = (lane % 32, lane / 32) holds A[r][16g .. 16g+15] and reads
// B[16g .. 16g+15][r] of each 32 x 32 x 32 step from LDS; D(i, j) lands in
// lane j + 32 ((i / 4) % 2), register (i / 8) 4 + i % 4.  The epilogue's
// per-channel constants and the staged rows' channel sums sit in LDS.
// TN (128 or 64) output steps per block; a wave covers TN / 2 of them.
// RES: the scaled fp32 output plus A.resid (its own instantiation: the
// residual's registers would lower the plain kernel's occupancy).
template <int TN, bool RES>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) conv_i8_kernel(ConvI8Args A) {
  constexpr int NI = TN / 64;  // 32-wide MFMA tiles per wave along time
  extern __shared__ __align__(16) int8_t conv_lds[];
  int8_t* Bw = conv_lds;                                          // [W4][kRowPitch]
  int* rs = reinterpret_cast<int*>(conv_lds + A.W4 * kRowPitch);  // [W4] channel sums
  int* cst = rs + A.W4;                                           // [kTileM] constant term
  float* scl = reinterpret_cast<float*>(cst + kTileM);            // [kTileM] scale
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int r = lane & 31, g = lane >> 5;
  const int wm = wv >> 1, wn = wv & 1;
  const uint3 tile = xcd_tile();  // neighbouring time tiles on one XCD
  const int64_t m0 = static_cast<int64_t>(tile.y) * kTileM;
  const int64_t nb = static_cast<int64_t>(tile.x) * TN;
  const int64_t b = tile.z;
  const uint8_t* xb = A.x + b * A.Cin * A.L;
  const int xz = (A.xzp ? static_cast<int>(A.xzp[0]) : 0) - 128;  // offset x zero point
  const uint32_t padb = static_cast<uint8_t>(static_cast<int8_t>(xz));
  const uint32_t padw = padb * 0x01010101u;
  // staged row 0 is source time a0 (padded time nb*s is source time nb*s - p0);
  // the window proper starts sh rows in
  const int64_t a = nb * A.s - A.p0;
  const int64_t a0 = A.aligned ? (a & ~int64_t{3}) : a;
  const int sh = static_cast<int>(a - a0);
  // v = acc + cst[co] - wz * S, with cst = K wz xz - xz sum(a) (+ bias) and
  // S = sum of b over the receptive field; the weight zero point is one
  // value for the tensor (every live row of wzo holds it)
  const int wz = A.wzo[0];
  if (tid < kTileM) {
    const int64_t co = m0 + tid;
    int c = 0;
    float sc = 0.0f;
    if (co < A.Cout) {
      c = static_cast<int>(A.Kreal) * wz * xz - xz * A.wsum[co];
      if (A.outf && A.qsa) {
        c += qbias_channel(A.qsa[0], A.qsw[0], A.qbias[co], &sc);
      } else if (A.outf) {
        if (A.bias) c += A.bias[co];
        sc = A.scale[A.scale_n > 1 ? co : 0];
      }
    }
    cst[tid] = c;
    scl[tid] = sc;
  }
  // A fragments straight from the fragment-ordered weights (no LDS): step
  // st = chunk * Kw + tap of row block m0 / 128 is 8 KB, wave row wm's four
  // fragments (ks, mi) 4 KB of it, lane l's 16 bytes of fragment q at
  // q * 1024 + 16 l.  A ring of three steps' fragments runs three steps
  // ahead; a load past the block's last step reads 0 (the buffer's range
  // check) and is never used.
  const int nch = static_cast<int>(A.CinP / kCinAlign), Kw = static_cast<int>(A.Kw);
  const int S = nch * Kw;
  const auto wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t*>(A.wT) + (m0 / kTileM) * static_cast<int64_t>(S) * 8192, 0, S * 8192,
      0x00020000);
  const uint32_t w_lane = static_cast<uint32_t>(wm * 4096 + lane * 16);
  auto lda = [&](int st, v4i (&f)[4]) {
    const uint32_t off = static_cast<uint32_t>(st) * 8192u + w_lane;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      f[q] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(wrs, off + 1024u * q, 0, 0));
  };
  // LDS offsets of this lane's B fragments: rows (wn*TN/2 + 32ni + r)*s +
  // tap*d + sh, columns 16g (+32 per k-step)
  int b_off[NI];
#pragma unroll
  for (int ni = 0; ni < NI; ++ni)
    b_off[ni] = ((wn * (TN / 2) + ni * 32 + r) * static_cast<int>(A.s) + sh) * kRowPitch + 16 * g;
  const int tap_step = static_cast<int>(A.d) * kRowPitch;
  const int ngrp = A.W4 / 4;  // groups of four staged rows
  const int nitems = static_cast<int>(ceil_div(ngrp, 16)) * 256;
  // 32-bit staging arithmetic (the host checks Cin * L < 2^31)
  const int Cin = static_cast<int>(A.Cin), Li = static_cast<int>(A.L);
  const uint32_t L = static_cast<uint32_t>(A.L);
  const int a0i = static_cast<int>(a0);
  // A chunk's window: item (tg, cg) = rows 4tg .. 4tg+3 x channels c0 +
  // 4cg .. 4cg+3.  A wave takes 4 channel groups x 16 consecutive time
  // groups: one channel of its items is 4 rows x 64 contiguous bytes (its
  // LDS writes meet 4-way bank conflicts, which cost little).  Then each
  // staged row's channel sum gains this chunk's share.
  // The window's loads are buffer loads, issued whatever the position (a
  // read outside x returns 0), with padding and missing channels chosen by
  // selects: no branch around a load, which keeps the compiler's wait counts
  // for the weight ring exact.
  const auto xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(xb), 0, Cin * Li,
                                                     0x00020000);
  auto stage = [&](int c0) {
    for (int it = tid; it < nitems; it += 256) {
      const int cg = (it >> 4) & 15, tg = (it & 15) + 16 * (it >> 8);
      const int ts = a0i + 4 * tg;
      const int ci0 = c0 + 4 * cg;
      uint32_t dw[4];
      if (A.aligned) {  // a dword is wholly inside the signal or wholly outside
        const bool in = ts >= 0 && ts < Li;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint32_t off = static_cast<uint32_t>(ci0 + e) * L + static_cast<uint32_t>(ts);
          asm volatile("" : "+v"(off));  // keeps the load unconditional
          const uint32_t ld = __builtin_amdgcn_raw_buffer_load_b32(xrs, off, 0, 0);
          dw[e] = ci0 + e < Cin ? (in ? (ld ^ 0x80808080u) : padw) : 0u;  // padding channels hold 0
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint32_t off = static_cast<uint32_t>(ci0 + e) * L + static_cast<uint32_t>(ts);
          asm volatile("" : "+v"(off));
          uint32_t v = 0;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int t = ts + q;
            const uint32_t ld = __builtin_amdgcn_raw_buffer_load_b8(xrs, off + q, 0, 0);
            v |= ((t >= 0 && t < Li) ? (ld ^ 0x80u) : padb) << (8 * q);
          }
          dw[e] = ci0 + e < Cin ? v : 0u;
        }
      }
      if (tg >= ngrp) continue;
      // 4 x 4 byte transpose (v_perm: bytes 0-3 from the second operand,
      // 4-7 from the first): word q = the four channels at time 4tg + q
      const uint32_t t01l = __builtin_amdgcn_perm(dw[1], dw[0], 0x05010400u);
      const uint32_t t01h = __builtin_amdgcn_perm(dw[1], dw[0], 0x07030602u);
      const uint32_t t23l = __builtin_amdgcn_perm(dw[3], dw[2], 0x05010400u);
      const uint32_t t23h = __builtin_amdgcn_perm(dw[3], dw[2], 0x07030602u);
      uint32_t* dst = reinterpret_cast<uint32_t*>(Bw + 4 * tg * kRowPitch + 4 * cg);
      dst[0] = __builtin_amdgcn_perm(t23l, t01l, 0x05040100u);
      dst[kRowPitch / 4] = __builtin_amdgcn_perm(t23l, t01l, 0x07060302u);
      dst[2 * kRowPitch / 4] = __builtin_amdgcn_perm(t23h, t01h, 0x05040100u);
      dst[3 * kRowPitch / 4] = __builtin_amdgcn_perm(t23h, t01h, 0x07060302u);
    }
    __syncthreads();
    for (int row = tid; row < A.W4; row += 256) {
      const int* p = reinterpret_cast<const int*>(Bw + row * kRowPitch);
      int sum = c0 == 0 ? 0 : rs[row];
#pragma unroll
      for (int k = 0; k < kCinAlign / 4; ++k) sum = __builtin_amdgcn_sdot4(p[k], 0x01010101, sum, false);
      rs[row] = sum;
    }
  };
  v16i acc[2][NI] = {};
  // one step's MFMAs: B fragments of the tap from the staged window
  auto mma = [&](int tap, const v4i (&f)[4]) {
    const int8_t* Bb = Bw + tap * tap_step;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      v4i bf[NI];
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        bf[ni] = *reinterpret_cast<const v4i*>(Bb + b_off[ni] + 32 * ks);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f[2 * ks + mi], bf[ni], acc[mi][ni], 0, 0, 0);
    }
  };
  v4i f0[4], f1[4], f2[4];
  lda(0, f0);
  lda(1, f1);
  lda(2, f2);
  int tap = 0, c0 = 0;
  // a chunk's first step stages its window (after every wave is done with
  // the previous one); the ring slot of step st is st % 3.  Every slot's
  // refill is issued whether or not its step exists (past the last step it
  // reads 0): a refill skipped on some path leaves the compiler's wait
  // counts for the other slots at "all loads", which drains the ring.
  auto run = [&](int st, v4i (&f)[4]) {
    if (st < S) {
      if (tap == 0) {
        if (st > 0) __syncthreads();
        stage(c0);
      }
      mma(tap, f);
      if (++tap == Kw) {
        tap = 0;
        c0 += kCinAlign;
      }
    }
    lda(st + 3, f);
  };
  for (int st = 0; st < S; st += 3) {
    run(st, f0);
    run(st + 1, f1);
    run(st + 2, f2);
  }
  __syncthreads();  // the last chunk's row sums, for the epilogue
  int zS[NI];  // wz * sum_k b_k of each of this lane's output columns
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int j = wn * (TN / 2) + 32 * ni + r;
    int S = 0;
    for (int tap = 0; tap < static_cast<int>(A.Kw); ++tap)
      S += rs[sh + j * static_cast<int>(A.s) + tap * static_cast<int>(A.d)];
    zS[ni] = wz * S;
  }
  // outputs from the block's corner, 32-bit byte offsets (the host checks
  // that a batch's output stays below 2 GiB); a block wholly inside the
  // output skips the per-element bounds checks
  const int64_t o_elem = (b * A.Cout + m0) * A.Lout + nb;
  char* ob = reinterpret_cast<char*>(A.outf ? static_cast<void*>(A.outf) : static_cast<void*>(A.out)) +
             4 * o_elem;
  const uint32_t lout4 = static_cast<uint32_t>(4 * A.Lout);
  const bool full = m0 + kTileM <= A.Cout && nb + TN <= A.Lout;
  const int c_rem = static_cast<int>(A.Cout - m0), l_rem = static_cast<int>(A.Lout - nb);
  const int lane_c = wm * 64 + 4 * g, lane_j = wn * (TN / 2) + r;
  const uint32_t lane_off = static_cast<uint32_t>(lane_c) * lout4 + 4u * static_cast<uint32_t>(lane_j);
  // the residual at the output's element offsets, through a buffer resource
  // over this batch's [Cout][Lout] (a read past it returns 0: rows past Cout
  // and columns past Lout of edge blocks are read but never stored)
  const auto rrs = __builtin_amdgcn_make_buffer_rsrc(
      RES ? const_cast<float*>(A.resid) + b * A.Cout * A.Lout : nullptr, 0,
      RES ? static_cast<int>(A.Cout * A.Lout * 4) : 0, 0x00020000);
  const uint32_t r_off = static_cast<uint32_t>(4 * (m0 * A.Lout + nb)) + lane_off;
  // This block's outputs are one numpy leaf of each of its rows (the
  // InstanceNorm that reads them sums its rows in numpy's pairwise order,
  // 8192-blocks of 64 leaves of 128 elements): its sum is formed here, in
  // that order, from the values as stored -- accumulator k of 8 sums the
  // elements 8 m + k, m = 0..15, one after another; then ((a0 + a1) + (a2 +
  // a3)) + ((a4 + a5) + (a6 + a7)).  A half (mi) of the tile, 64 rows x 128
  // steps, goes through LDS (kLeafPitch floats a row: the two rows a store
  // instruction writes fall 32 banks apart), where four threads a row each
  // sum two accumulators from their own addresses and two shuffles form the
  // tree.
  const bool leafy = TN == 128 && A.leaf && static_cast<int64_t>(tile.x) < A.nleaf;
  float* const lt = reinterpret_cast<float*>(conv_lds + conv_leaf_off(A.W4));  // [64][kLeafPitch]
  auto epilogue = [&](auto full_tile) {
    constexpr bool kFull = decltype(full_tile)::value;
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
      // the stored values (for the leaf sums), and before them the residual
      // of this half of the lane's outputs, all its loads issued before the
      // first store (a load after a store to a possibly aliasing address
      // would wait for it: one memory round trip per element)
      float yv[16][NI];
      if constexpr (RES) {
#pragma unroll
        for (int reg = 0; reg < 16; ++reg) {
          const int cr = 32 * mi + 8 * (reg / 4) + (reg % 4);
          const uint32_t roff = r_off + static_cast<uint32_t>(cr) * lout4;
#pragma unroll
          for (int ni = 0; ni < NI; ++ni)
            yv[reg][ni] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(rrs, roff + 128u * ni, 0, 0));
        }
      }
#pragma unroll
      for (int reg = 0; reg < 16; ++reg) {
        const int cr = 32 * mi + 8 * (reg / 4) + (reg % 4);  // constant once unrolled
        const int cl = lane_c + cr;
        if (!kFull && cl >= c_rem) continue;
        const int c = cst[cl];
        const float sc = scl[cl];
        const uint32_t roff = lane_off + static_cast<uint32_t>(cr) * lout4;
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
          if (!kFull && lane_j + 32 * ni >= l_rem) continue;
          const int v = acc[mi][ni][reg] + c - zS[ni];
          char* dst = ob + (roff + 128u * ni);
          if constexpr (RES) {
            yv[reg][ni] = static_cast<float>(v) * sc + yv[reg][ni];
            *reinterpret_cast<float*>(dst) = yv[reg][ni];
          } else if (A.outf) {
            yv[reg][ni] = static_cast<float>(v) * sc;
            *reinterpret_cast<float*>(dst) = yv[reg][ni];
          } else {
            *reinterpret_cast<int*>(dst) = v;
          }
        }
      }
      if constexpr (TN == 128) {
        if (leafy) {  // block-uniform: every wave meets the barriers
#pragma unroll
          for (int reg = 0; reg < 16; ++reg) {
            const int rl = wm * 32 + 8 * (reg / 4) + 4 * g + (reg % 4);
#pragma unroll
            for (int ni = 0; ni < NI; ++ni)
              lt[rl * kLeafPitch + wn * 64 + 32 * ni + r] = yv[reg][ni];
          }
          __syncthreads();
          const int rl = tid >> 2, q = tid & 3;  // row rl, accumulators 2q and 2q + 1
          const float* src = lt + rl * kLeafPitch + 2 * q;
          float a0 = src[0], a1 = src[1];
#pragma unroll
          for (int m = 1; m < 16; ++m) {
            a0 = a0 + src[8 * m];
            a1 = a1 + src[8 * m + 1];
          }
          float p = a0 + a1;
          p = p + __shfl_xor(p, 1, 64);
          p = p + __shfl_xor(p, 2, 64);
          const int cl = (rl >> 5) * 64 + 32 * mi + (rl & 31);
          if (q == 0 && cl < c_rem) A.leaf[(b * A.Cout + m0 + cl) * A.nleaf + tile.x] = p;
          if (mi == 0) __syncthreads();  // (the next half reuses the area)
        }
      }
    }
  };
  if (full) epilogue(std::true_type{});
  else epilogue(std::false_type{});
}

}  // namespace i8conv
using namespace i8conv;

static int64_t conv_window(int64_t tn, int64_t stride, int64_t dilation, int64_t K) {
  return (tn - 1) * stride + (K - 1) * dilation + 1;
}

// Staged rows: the window plus up to 3 rows of alignment slack, in groups of 4.
static int64_t conv_rows(int64_t tn, int64_t stride, int64_t dilation, int64_t K) {
  return ceil_div(conv_window(tn, stride, dilation, K) + 3, 4) * 4;
}

// LDS of a block: the staged rows and their channel sums, the per-channel
// epilogue constants.
static size_t conv_lds(int64_t rows) {
  return static_cast<size_t>(rows * (kRowPitch + 4) + 2 * kTileM * 4);
}

// The time tile (128, else 64) whose block fits 64 KB of LDS; 0 if neither does.
static int conv_tile_n(int64_t stride, int64_t dilation, int64_t K) {
  for (int tn : {128, 64})
    if (conv_lds(conv_rows(tn, stride, dilation, K)) <= 65536) return tn;
  return 0;
}

// The launch's time tile: 128 when its blocks still give every CU two (the
// kernel is latency-bound and three blocks share a CU), else 64 for twice
// the blocks.  Measured on the 128-id graph (whose convolutions run at
// 240 .. 431,000 steps): 128 everywhere 39.6 ms, 64 everywhere 38.4 ms, and
// 64 everywhere 7% slower on [1,128,431000] alone.
static int conv_launch_tile(int64_t stride, int64_t dilation, int64_t K, int64_t N,
                            int64_t CoutP, int64_t Lout) {
  const int tn = conv_tile_n(stride, dilation, K);
  const int64_t cus = ctx().num_cus > 0 ? ctx().num_cus : 256;
  if (tn == 128 && N * (CoutP / kTileM) * ceil_div(Lout, 128) < 2 * cus &&
      conv_lds(conv_rows(64, stride, dilation, K)) <= 65536)
    return 64;
  return tn;
}

// The allocation-free entry point's workspace: a file-scope device array of
// a fixed size (2.4x the largest the Kokoro graph's convolutions need,
// 3.4 MiB), which each device holds from the library's first use of it until
// the process ends.  Its host-side name is only a stand-in for the symbol:
// the device address comes from hipGetSymbolAddress, taken once per device
// by conv_i8_scratch_setup (called from kk_init with the device current) and
// kept in g_scratch; kernels and copies only ever see that address.
constexpr size_t kNoAllocBytes = size_t{8} << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];
constexpr int kMaxDevices = 64;
static void* g_scratch[kMaxDevices];

int conv_i8_scratch_setup(int device) {
  if (device < 0 || device >= kMaxDevices)
    return set_error(KK_E_UNSUPPORTED, "device %d beyond the %d the library tracks", device,
                     kMaxDevices);
  if (g_scratch[device]) return KK_OK;
  void* p = nullptr;
  KK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  if (!p) return set_error(KK_E_HIP, "hipGetSymbolAddress gave no address for the conv scratch");
  g_scratch[device] = p;
  return KK_OK;
}

// Byte offsets of a call's workspace: the re-laid weights wT, then four
// per-channel int32/fp32 arrays (weight sums, offset zero points, scale,
// quantised bias), each 256-byte aligned.
struct ConvWs {
  int64_t wT, wsum, wzo, qs, qb, total;
};
static ConvWs conv_ws_layout(int64_t Cout, int64_t Cin, int64_t Kw) {
  const int64_t CinP = ceil_div(Cin, kCinAlign) * kCinAlign;
  const int64_t CoutP = ceil_div(Cout, kTileM) * kTileM;
  auto up = [](int64_t n) { return ceil_div(n, 256) * 256; };
  ConvWs L{};
  L.wT = 0;
  L.wsum = L.wT + up(CoutP * Kw * CinP);
  L.wzo = L.wsum + up(CoutP * 4);
  L.qs = L.wzo + up(CoutP * 4);
  L.qb = L.qs + up(CoutP * 4);
  L.total = L.qb + up(CoutP * 4);
  return L;
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
  if (ceil_div(Cout, kTileM) * kTileM * Lout * 4 >= (int64_t{1} << 31) ||  // 32-bit offsets
      (Cin + 64) * (L + 64) >= (int64_t{1} << 31))
    return set_error(KK_E_UNSUPPORTED, "%s: Cout * Lout or Cin * L too large", who);
  // a block's input window must fit LDS beside the weight double buffer
  if (conv_tile_n(stride, dilation, K) == 0)
    return set_error(KK_E_UNSUPPORTED, "%s: stride %d / dilation %d / kernel %lld: input window "
                     "of %lld rows does not fit LDS", who, stride, dilation, (long long)K,
                     (long long)conv_window(64, stride, dilation, K));
  *lout = Lout;
  return KK_OK;
}

// Every entry point: `outf` set gives the scaled fp32 form; `fixed_ws`, when
// given, is the workspace (conv_ws_layout(...).total bytes, checked by the
// caller) instead of one from the pool.
static int conv_integer_run(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                     const kk_tensor* x_zp, const kk_tensor* w_zp, const kk_tensor* bias,
                     const kk_tensor* scale, int stride, int dilation, int pad0, int pad1,
                     bool outf, const kk_tensor* qb_sa = nullptr, const kk_tensor* qb_sw = nullptr,
                     const kk_tensor* qb_bias = nullptr, void* fixed_ws = nullptr,
                     const kk_tensor* resid = nullptr, const kk_tensor* packed = nullptr,
                     const kk_tensor* leaves = nullptr) {
  const int64_t N = x->shape[0], Cin = x->shape[1], L = x->shape[2];
  const int64_t Cout = w->shape[0], Kw = w->shape[2];
  const int64_t Lout = out->shape[2];
  const int64_t CinP = ceil_div(Cin, kCinAlign) * kCinAlign;
  const int64_t CoutP = ceil_div(Cout, kTileM) * kTileM;
  const ConvWs lay = conv_ws_layout(Cout, Cin, Kw);
  // packed weights (kk_conv_integer_pack) hold wT, wsum and wzo already
  void* ws = packed ? packed->data : fixed_ws;
  const bool own_ws = !ws;
  if (own_ws) KK_TRY(kk_alloc(static_cast<size_t>(lay.total), &ws));
  char* base = static_cast<char*>(ws);
  int8_t* wT = reinterpret_cast<int8_t*>(base + lay.wT);
  int32_t* wsum = reinterpret_cast<int32_t*>(base + lay.wsum);
  int32_t* wzo = reinterpret_cast<int32_t*>(base + lay.wzo);
  QBias qb{};
  if (qb_sa && !packed) {
    qb.sa = static_cast<const float*>(qb_sa->data);
    qb.sw = static_cast<const float*>(qb_sw->data);
    qb.bias = static_cast<const float*>(qb_bias->data);
    qb.scale = reinterpret_cast<float*>(base + lay.qs);
    qb.ibias = reinterpret_cast<int32_t*>(base + lay.qb);
  }
  hipStream_t st = ctx().stream;
  int rc = KK_OK;
  if (!packed) {
    KK_LAUNCH(conv_i8_wprep, dim3(static_cast<unsigned>(CoutP)), dim3(256), 0, st, w->data,
                       w->dtype, w_zp ? w_zp->data : nullptr, w_zp ? w_zp->dtype : 0,
                       w_zp ? numel(w_zp) : 0, wT, wsum, wzo, Cout, Cin, Kw, CinP, qb);
    rc = check_launch("conv_i8_wprep");
  }
  if (rc == KK_OK) {
    ConvI8Args A{};
    A.wT = wT; A.wsum = wsum; A.wzo = wzo;
    A.x = static_cast<const uint8_t*>(x->data);
    A.xzp = x_zp ? static_cast<const uint8_t*>(x_zp->data) : nullptr;
    if (outf && packed && qb_sa) {
      A.outf = static_cast<float*>(out->data);
      A.qsa = static_cast<const float*>(qb_sa->data);
      A.qsw = static_cast<const float*>(qb_sw->data);
      A.qbias = static_cast<const float*>(qb_bias->data);
    } else if (outf && qb.scale) {
      A.outf = static_cast<float*>(out->data);
      A.bias = qb.ibias;
      A.scale = qb.scale;
      A.scale_n = Cout;
    } else if (outf) {
      A.outf = static_cast<float*>(out->data);
      A.bias = bias ? static_cast<const int32_t*>(bias->data) : nullptr;
      A.scale = static_cast<const float*>(scale->data);
      A.scale_n = numel(scale);
    } else {
      A.out = static_cast<int32_t*>(out->data);
    }
    A.Cout = Cout; A.Cin = Cin; A.CinP = CinP; A.Kw = Kw; A.s = stride; A.d = dilation;
    A.L = L; A.p0 = pad0; A.Lout = Lout; A.Kreal = Cin * Kw;
    A.resid = resid ? static_cast<const float*>(resid->data) : nullptr;
    A.aligned = (L % 4 == 0) && (reinterpret_cast<uintptr_t>(x->data) % 4 == 0);
    // leaf sums need the 128-step tiles (checked to fit by the caller)
    const int tn = leaves ? 128 : conv_launch_tile(stride, dilation, Kw, N, CoutP, Lout);
    if (leaves) {
      A.leaf = static_cast<float*>(leaves->data);
      A.nleaf = (Lout / 8192) * 64;
    }
    A.W4 = static_cast<int>(conv_rows(tn, stride, dilation, Kw));
    const dim3 grid(static_cast<unsigned>(ceil_div(Lout, tn)),
                    static_cast<unsigned>(CoutP / kTileM), static_cast<unsigned>(N));
    rc = check_xcd_grid(grid, "ConvInteger");
    if (rc == KK_OK) {
      const size_t lds = A.leaf ? static_cast<size_t>(conv_leaf_off(A.W4) + kLeafBytes)
                                : conv_lds(A.W4);
      if (A.resid) {
        if (tn == 128) KK_LAUNCH((conv_i8_kernel<128, true>), grid, dim3(256), lds, st, A);
        else KK_LAUNCH((conv_i8_kernel<64, true>), grid, dim3(256), lds, st, A);
      } else {
        if (tn == 128) KK_LAUNCH((conv_i8_kernel<128, false>), grid, dim3(256), lds, st, A);
        else KK_LAUNCH((conv_i8_kernel<64, false>), grid, dim3(256), lds, st, A);
      }
      rc = check_launch("conv_i8_kernel");
    }
  }
  if (own_ws) kk_free(ws);  // stream order keeps the workspace alive for the kernels
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

}  // extern "C"

// The residual of the _add entry points: fp32, contiguous, shaped like out.
static int check_resid(const kk_tensor* out, const kk_tensor* resid, const char* who) {
  KK_TRY(check_tensor(resid, "resid"));
  bool same = resid->rank == out->rank;
  for (int i = 0; same && i < out->rank; ++i) same = resid->shape[i] == out->shape[i];
  if (resid->dtype != KK_F32 || !is_contiguous(resid) || !same)
    return set_error(KK_E_ARG, "%s: resid must be fp32, contiguous and shaped like out", who);
  return KK_OK;
}

static int scaled_entry(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                        const kk_tensor* x_zp, const kk_tensor* w_zp, const kk_tensor* bias,
                        const kk_tensor* scale, const kk_tensor* resid, int stride, int dilation,
                        int pad0, int pad1, int group, const char* who) {
  int64_t Lout = 0;
  KK_TRY(check_conv_integer(out, x, w, x_zp, w_zp, stride, dilation, pad0, pad1, group, KK_F32,
                            who, &Lout));
  if (resid) KK_TRY(check_resid(out, resid, who));
  const int64_t Cout = w->shape[0];
  KK_TRY(check_tensor(scale, "scale"));
  if (scale->dtype != KK_F32 || !is_contiguous(scale) ||
      (numel(scale) != 1 && numel(scale) != Cout))
    return set_error(KK_E_ARG, "%s: scale must be fp32 with 1 or Cout values", who);
  if (bias) {
    KK_TRY(check_tensor(bias, "bias"));
    if (bias->dtype != KK_I32 || !is_contiguous(bias) || numel(bias) != Cout)
      return set_error(KK_E_ARG, "%s: bias must be int32 with Cout values", who);
  }
  if (numel(out) == 0) return KK_OK;
  if (x->shape[1] * w->shape[2] == 0)
    return set_error(KK_E_UNSUPPORTED, "%s: empty reduction", who);
  return conv_integer_run(out, x, w, x_zp, w_zp, bias, scale, stride, dilation, pad0, pad1, true,
                          nullptr, nullptr, nullptr, nullptr, resid);
}

extern "C" {

int kk_conv_integer_scaled(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                           const kk_tensor* x_zp, const kk_tensor* w_zp, const kk_tensor* bias,
                           const kk_tensor* scale, int stride, int dilation, int pad0, int pad1,
                           int group) {
  return scaled_entry(out, x, w, x_zp, w_zp, bias, scale, nullptr, stride, dilation, pad0, pad1,
                      group, "kk_conv_integer_scaled");
}

int kk_conv_integer_scaled_add(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                               const kk_tensor* x_zp, const kk_tensor* w_zp, const kk_tensor* bias,
                               const kk_tensor* scale, const kk_tensor* resid, int stride,
                               int dilation, int pad0, int pad1, int group) {
  if (!resid) return set_error(KK_E_ARG, "kk_conv_integer_scaled_add: resid is required");
  return scaled_entry(out, x, w, x_zp, w_zp, bias, scale, resid, stride, dilation, pad0, pad1,
                      group, "kk_conv_integer_scaled_add");
}

}  // extern "C"

// The checks of kk_conv_integer_scaled_qbias (and its allocation-free form):
// KK_OK to run, or an error; *empty when there is nothing to compute.
static int check_qbias(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                       const kk_tensor* x_zp, const kk_tensor* w_zp, const kk_tensor* bias,
                       const kk_tensor* scale_a, const kk_tensor* scale_w, int stride, int dilation,
                       int pad0, int pad1, int group, const char* who, bool* empty) {
  int64_t Lout = 0;
  KK_TRY(check_conv_integer(out, x, w, x_zp, w_zp, stride, dilation, pad0, pad1, group, KK_F32,
                            who, &Lout));
  const int64_t Cout = w->shape[0];
  const kk_tensor* one[2] = {scale_a, scale_w};
  for (const kk_tensor* t : one) {
    KK_TRY(check_tensor(t, "scale"));
    if (t->dtype != KK_F32 || numel(t) != 1)
      return set_error(KK_E_ARG, "%s: scale_a and scale_w are one fp32 each", who);
  }
  KK_TRY(check_tensor(bias, "bias"));
  if (bias->dtype != KK_F32 || !is_contiguous(bias) || numel(bias) != Cout)
    return set_error(KK_E_ARG, "%s: bias must be fp32 with Cout values", who);
  *empty = numel(out) == 0;
  if (!*empty && x->shape[1] * w->shape[2] == 0)
    return set_error(KK_E_UNSUPPORTED, "%s: empty reduction", who);
  return KK_OK;
}

// What each packed buffer was made from (kk_conv_integer_pack), by its
// device address: a call must pass the same weight tensor (address, shape,
// dtype) and the same zero-point tensor (address, dtype) the pack read, so
// a buffer packed for another weight or zero point is refused, not used.
struct PackRecord {
  const void* w;
  int64_t cout, cin, k;
  int w_dt;
  const void* zp;
  int zp_dt;
};
static std::mutex g_pack_mu;
static std::unordered_map<const void*, PackRecord> g_packs;

void kk::conv_i8_forget_pack(const void* p) {
  std::lock_guard<std::mutex> lock(g_pack_mu);
  g_packs.erase(p);
}

static PackRecord pack_record(const kk_tensor* w, const kk_tensor* w_zp) {
  return PackRecord{w->data, w->shape[0], w->shape[1], w->shape[2], w->dtype,
                    w_zp ? w_zp->data : nullptr, w_zp ? w_zp->dtype : -1};
}

extern "C" {

int kk_conv_integer_scaled_qbias(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                                 const kk_tensor* x_zp, const kk_tensor* w_zp,
                                 const kk_tensor* bias, const kk_tensor* scale_a,
                                 const kk_tensor* scale_w, int stride, int dilation, int pad0,
                                 int pad1, int group) {
  bool empty = false;
  KK_TRY(check_qbias(out, x, w, x_zp, w_zp, bias, scale_a, scale_w, stride, dilation, pad0, pad1,
                     group, "kk_conv_integer_scaled_qbias", &empty));
  if (empty) return KK_OK;
  return conv_integer_run(out, x, w, x_zp, w_zp, nullptr, nullptr, stride, dilation, pad0, pad1,
                          true, scale_a, scale_w, bias);
}

int kk_conv_integer_scaled_qbias_add(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                                     const kk_tensor* x_zp, const kk_tensor* w_zp,
                                     const kk_tensor* bias, const kk_tensor* scale_a,
                                     const kk_tensor* scale_w, const kk_tensor* resid, int stride,
                                     int dilation, int pad0, int pad1, int group) {
  const char* who = "kk_conv_integer_scaled_qbias_add";
  bool empty = false;
  KK_TRY(check_qbias(out, x, w, x_zp, w_zp, bias, scale_a, scale_w, stride, dilation, pad0, pad1,
                     group, who, &empty));
  if (!resid) return set_error(KK_E_ARG, "%s: resid is required", who);
  KK_TRY(check_resid(out, resid, who));
  if (empty) return KK_OK;
  return conv_integer_run(out, x, w, x_zp, w_zp, nullptr, nullptr, stride, dilation, pad0, pad1,
                          true, scale_a, scale_w, bias, nullptr, resid);
}

int kk_conv_integer_packed_bytes(int64_t cout, int64_t cin, int64_t k, int64_t* bytes) {
  if (!bytes || cout <= 0 || cin <= 0 || k <= 0)
    return set_error(KK_E_ARG, "kk_conv_integer_packed_bytes: positive sizes and an output");
  *bytes = conv_ws_layout(cout, cin, k).qs;  // wT, wsum and wzo
  return KK_OK;
}

// The packed weights' checks: uint8, contiguous, 256-byte aligned, sized
// for w's shape; with `made_from`, also that the pack was made from this w
// and w_zp.
static int check_packed(const kk_tensor* packed, const kk_tensor* w, const char* who,
                        const kk_tensor* w_zp = nullptr, bool made_from = false) {
  KK_TRY(check_tensor(packed, "packed"));
  const int64_t need = conv_ws_layout(w->shape[0], w->shape[1], w->shape[2]).qs;
  if (packed->dtype != KK_U8 || !is_contiguous(packed) || numel(packed) != need ||
      reinterpret_cast<uintptr_t>(packed->data) % 256 != 0)
    return set_error(KK_E_ARG, "%s: packed must be %lld contiguous, 256-byte aligned uint8 bytes",
                     who, (long long)need);
  if (made_from) {
    const PackRecord want = pack_record(w, w_zp);
    std::lock_guard<std::mutex> lock(g_pack_mu);
    auto it = g_packs.find(packed->data);
    if (it == g_packs.end())
      return set_error(KK_E_ARG, "%s: packed was not made by kk_conv_integer_pack", who);
    const PackRecord& r = it->second;
    if (r.w != want.w || r.cout != want.cout || r.cin != want.cin || r.k != want.k ||
        r.w_dt != want.w_dt)
      return set_error(KK_E_ARG, "%s: packed was made from another weight tensor", who);
    if (r.zp != want.zp || r.zp_dt != want.zp_dt)
      return set_error(KK_E_ARG, "%s: packed was made with another weight zero point", who);
  }
  return KK_OK;
}

int kk_conv_integer_pack(const kk_tensor* packed, const kk_tensor* w, const kk_tensor* w_zp) {
  const char* who = "kk_conv_integer_pack";
  KK_TRY(require_ready());
  KK_TRY(check_tensor(w, "w"));
  if (w->rank != 3 || !(w->dtype == KK_U8 || w->dtype == KK_I8) || !is_contiguous(w) ||
      numel(w) == 0)
    return set_error(KK_E_ARG, "%s: w must be a non-empty contiguous uint8/int8 [Cout, Cin, K]",
                     who);
  if (w_zp) {
    KK_TRY(check_tensor(w_zp, "w_zp"));
    if (!(w_zp->dtype == KK_U8 || w_zp->dtype == KK_I8 || w_zp->dtype == KK_I32) ||
        numel(w_zp) != 1)
      return set_error(KK_E_ARG, "%s: w_zp must be one uint8/int8/int32", who);
  }
  KK_TRY(check_packed(packed, w, who));
  const int64_t Cout = w->shape[0], Cin = w->shape[1], Kw = w->shape[2];
  const int64_t CinP = ceil_div(Cin, kCinAlign) * kCinAlign;
  const int64_t CoutP = ceil_div(Cout, kTileM) * kTileM;
  const ConvWs lay = conv_ws_layout(Cout, Cin, Kw);
  {
    std::lock_guard<std::mutex> lock(g_pack_mu);
    g_packs[packed->data] = pack_record(w, w_zp);
  }
  char* base = static_cast<char*>(packed->data);
  KK_LAUNCH(conv_i8_wprep, dim3(static_cast<unsigned>(CoutP)), dim3(256), 0, ctx().stream,
                     w->data, w->dtype, w_zp ? w_zp->data : nullptr, w_zp ? w_zp->dtype : 0,
                     w_zp ? numel(w_zp) : 0, reinterpret_cast<int8_t*>(base + lay.wT),
                     reinterpret_cast<int32_t*>(base + lay.wsum),
                     reinterpret_cast<int32_t*>(base + lay.wzo), Cout, Cin, Kw, CinP, QBias{});
  return check_launch("conv_i8_wprep");
}

int kk_conv_integer_scaled_qbias_packed(const kk_tensor* out, const kk_tensor* x,
                                        const kk_tensor* w, const kk_tensor* packed,
                                        const kk_tensor* x_zp, const kk_tensor* w_zp,
                                        const kk_tensor* bias, const kk_tensor* scale_a,
                                        const kk_tensor* scale_w, const kk_tensor* resid,
                                        int stride, int dilation, int pad0, int pad1, int group) {
  const char* who = "kk_conv_integer_scaled_qbias_packed";
  bool empty = false;
  KK_TRY(check_qbias(out, x, w, x_zp, w_zp, bias, scale_a, scale_w, stride, dilation, pad0, pad1,
                     group, who, &empty));
  KK_TRY(check_packed(packed, w, who, w_zp, true));
  if (resid) KK_TRY(check_resid(out, resid, who));
  if (empty) return KK_OK;
  return conv_integer_run(out, x, w, x_zp, w_zp, nullptr, nullptr, stride, dilation, pad0, pad1,
                          true, scale_a, scale_w, bias, nullptr, resid, packed);
}

int kk_conv_integer_scaled_qbias_packed_leaves(
    const kk_tensor* out, const kk_tensor* x, const kk_tensor* w, const kk_tensor* packed,
    const kk_tensor* x_zp, const kk_tensor* w_zp, const kk_tensor* bias, const kk_tensor* scale_a,
    const kk_tensor* scale_w, const kk_tensor* resid, const kk_tensor* leaves, int stride,
    int dilation, int pad0, int pad1, int group) {
  const char* who = "kk_conv_integer_scaled_qbias_packed_leaves";
  bool empty = false;
  KK_TRY(check_qbias(out, x, w, x_zp, w_zp, bias, scale_a, scale_w, stride, dilation, pad0, pad1,
                     group, who, &empty));
  KK_TRY(check_packed(packed, w, who, w_zp, true));
  if (resid) KK_TRY(check_resid(out, resid, who));
  if (leaves) {
    KK_TRY(check_tensor(leaves, "leaves"));
    const int64_t rows = out->shape[0] * out->shape[1], Lout = out->shape[2];
    const int64_t nleaf = (Lout / 8192) * 64;
    if (nleaf == 0)
      return set_error(KK_E_ARG, "%s: rows of %lld steps hold no whole 8192-block", who,
                       (long long)Lout);
    if (leaves->dtype != KK_F32 || !is_contiguous(leaves) || numel(leaves) != rows * nleaf)
      return set_error(KK_E_ARG, "%s: leaves must be %lld contiguous fp32 values", who,
                       (long long)(rows * nleaf));
    if (conv_leaf_off(static_cast<int>(conv_rows(128, stride, dilation, w->shape[2]))) +
            kLeafBytes > 65536)
      return set_error(KK_E_UNSUPPORTED, "%s: the 128-step tile's window does not fit LDS", who);
  }
  if (empty) return KK_OK;
  KK_TRY(conv_integer_run(out, x, w, x_zp, w_zp, nullptr, nullptr, stride, dilation, pad0, pad1,
                          true, scale_a, scale_w, bias, nullptr, resid, packed, leaves));
  if (leaves) leaf_record(leaves->data, out->data, out->shape[0] * out->shape[1], out->shape[2]);
  return KK_OK;
}

int kk_conv_integer_scaled_qbias_noalloc(const kk_tensor* out, const kk_tensor* x,
                                         const kk_tensor* w, const kk_tensor* x_zp,
                                         const kk_tensor* w_zp, const kk_tensor* bias,
                                         const kk_tensor* scale_a, const kk_tensor* scale_w,
                                         int stride, int dilation, int pad0, int pad1, int group) {
  const char* who = "kk_conv_integer_scaled_qbias_noalloc";
  bool empty = false;
  KK_TRY(check_qbias(out, x, w, x_zp, w_zp, bias, scale_a, scale_w, stride, dilation, pad0, pad1,
                     group, who, &empty));
  const ConvWs lay = conv_ws_layout(w->shape[0], w->shape[1], w->shape[2]);
  if (lay.total > static_cast<int64_t>(kNoAllocBytes))
    return set_error(KK_E_UNSUPPORTED,
                     "%s: Cout %lld x Cin %lld x K %lld needs a %lld-byte workspace, beyond the "
                     "%zu bytes of the allocation-free scratch", who, (long long)w->shape[0],
                     (long long)w->shape[1], (long long)w->shape[2], (long long)lay.total,
                     kNoAllocBytes);
  const int dev = ctx().device;
  if (dev < 0 || dev >= kMaxDevices || !g_scratch[dev])
    return set_error(KK_E_STATE, "%s: the scratch of device %d is not set up", who, dev);
  if (empty) return KK_OK;
  return conv_integer_run(out, x, w, x_zp, w_zp, nullptr, nullptr, stride, dilation, pad0, pad1,
                          true, scale_a, scale_w, bias, g_scratch[dev]);
}

}  // extern "C"
