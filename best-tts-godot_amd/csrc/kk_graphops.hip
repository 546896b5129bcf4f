// The rest of the Kokoro graph's device ops: DynamicQuantizeLinear, the
// DynamicQuantizeLSTM recurrence, STFT, Resize, Pad, CumSum and ScatterND.
#include <algorithm>
#include <cmath>
#include <vector>

#include "kk_internal.h"

namespace kk {

// --------------------------------------------------- DynamicQuantizeLinear
// Stage 1: per-block (min, max) partials.  Stage 2: every block folds them,
// derives scale and zero point in double exactly as the reference does
// (ref_runtime.py:106-116) and writes its share of the bytes.  Both stages
// read x as float4 when it is 16-byte aligned (stage 1 with cached loads,
// which stage 2 finds in the L2 for the graph's activations); the quantised
// bytes leave four at a time.
constexpr int kDqlBlocks = 256;  // stage-1 blocks at most (one partial a thread of a stage-2 block)


// One block folds the partials and derives scale and zero point in double
// exactly as the reference does; params = (scale, zero point) as floats.
constexpr int kDqlFoldThreads = 1024;

// only_if: the launch does nothing unless *only_if == epoch (the value a
// pass of the same call stores there).  clear: also keeps the folded (min,
// max) in params[1] and zeroes *clear, the flag a later pass sets (to
// epoch) when one of its values falls outside that range.
__global__ void __launch_bounds__(kDqlFoldThreads) dql_fold(const float2* __restrict__ part,
                                                            int npart, float2* __restrict__ params,
                                                            float* __restrict__ scale_out,
                                                            uint8_t* __restrict__ zp_out,
                                                            const int* __restrict__ only_if,
                                                            int* __restrict__ clear, int epoch) {
  if (only_if && *only_if != epoch) return;
  __shared__ float smin[kDqlFoldThreads / 64], smax[kDqlFoldThreads / 64];
  float lo = INFINITY, hi = -INFINITY;
  for (int i = threadIdx.x; i < npart; i += blockDim.x) {
    lo = fminf(lo, part[i].x);
    hi = fmaxf(hi, part[i].y);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, off, 64));
    hi = fmaxf(hi, __shfl_xor(hi, off, 64));
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) { smin[w] = lo; smax[w] = hi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float fmn = smin[0], fmx = smax[0];
    for (int k = 1; k < kDqlFoldThreads / 64; ++k) {
      fmn = fminf(fmn, smin[k]);
      fmx = fmaxf(fmx, smax[k]);
    }
    params[0] = dql_params(fmn, fmx, scale_out, zp_out);
    if (clear) {
      params[1] = make_float2(fmn, fmx);
      *clear = 0;
    }
  }
}


// Stage 1: at most kDqlBlocks blocks each take the (min, max) of their
// grid-stride share, four float4 loads in flight a thread, and store it.
// No block waits for another and none counts in (a count that every block
// of a large grid increments serialises on its one address: 2048 blocks
// took 40 us): the stage-2 blocks fold the partials themselves.
__global__ void __launch_bounds__(256) dql_minmax_part(const float* __restrict__ x, int64_t n,
                                                        float2* __restrict__ part, int vec) {
  __shared__ float smin[4], smax[4];
  float lo = INFINITY, hi = -INFINITY;
  const int64_t tid = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  const int64_t nthreads = static_cast<int64_t>(gridDim.x) * blockDim.x;
  int64_t head = 0;
  if (vec) {
    constexpr int kU = 4;
    const int64_t n4 = n / 4;
    const float x0 = x[0];  // (past the end a slot holds x[0], which moves neither extreme)
    for (int64_t i0 = tid; i0 < n4; i0 += nthreads * kU) {
      float4 v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int64_t i = i0 + u * nthreads;
        v[u] = i < n4 ? *reinterpret_cast<const float4*>(x + 4 * i)  // read again by stage 2
                      : make_float4(x0, x0, x0, x0);
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        lo = fminf(lo, fminf(fminf(v[u].x, v[u].y), fminf(v[u].z, v[u].w)));
        hi = fmaxf(hi, fmaxf(fmaxf(v[u].x, v[u].y), fmaxf(v[u].z, v[u].w)));
      }
    }
    head = 4 * n4;
  }
  for (int64_t i = head + tid; i < n; i += nthreads) {
    const float v = x[i];
    lo = fminf(lo, v);
    hi = fmaxf(hi, v);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, off, 64));
    hi = fmaxf(hi, __shfl_xor(hi, off, 64));
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) { smin[w] = lo; smax[w] = hi; }
  __syncthreads();
  if (threadIdx.x == 0)
    part[blockIdx.x] = make_float2(fminf(fminf(smin[0], smin[1]), fminf(smin[2], smin[3])),
                                   fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3])));
}

// Stage 2: every block folds the npart (<= 256) partials (min and max do
// not depend on the order, so every block finds the same scale and zero
// point; block 0 stores them) and quantises its grid-stride share.
__global__ void __launch_bounds__(256) dql_quantize_fold(const float* __restrict__ x, int64_t n,
                                                          const float2* __restrict__ part, int npart,
                                                          float* __restrict__ scale_out,
                                                          uint8_t* __restrict__ zp_out,
                                                          uint8_t* __restrict__ y, int vec) {
  __shared__ float smin[4], smax[4];
  __shared__ float2 pz_s;
  float lo = INFINITY, hi = -INFINITY;
  if (static_cast<int>(threadIdx.x) < npart) {
    const float2 q = part[threadIdx.x];
    lo = q.x;
    hi = q.y;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, off, 64));
    hi = fmaxf(hi, __shfl_xor(hi, off, 64));
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) { smin[w] = lo; smax[w] = hi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float sc;
    uint8_t zq;
    pz_s = dql_params(fminf(fminf(smin[0], smin[1]), fminf(smin[2], smin[3])),
                      fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3])), &sc, &zq);
    if (blockIdx.x == 0) {
      *scale_out = sc;
      *zp_out = zq;
    }
  }
  __syncthreads();
  const float sc = pz_s.x, z = pz_s.y;
  const KkDivisor dsc = kk_divisor(sc);
  const int64_t tid = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  const int64_t nthreads = static_cast<int64_t>(gridDim.x) * blockDim.x;
  int64_t head = 0;
  if (vec) {
    const int64_t n4 = n / 4;
    for (int64_t i = tid; i < n4; i += nthreads) {
      const uint32_t q = dql_bytes4(ld_stream4(x + 4 * i), dsc, z);
      __builtin_nontemporal_store(q, reinterpret_cast<uint32_t*>(y) + i);
    }
    head = 4 * n4;
  }
  for (int64_t i = head + tid; i < n; i += nthreads) y[i] = static_cast<uint8_t>(dql_byte(x[i], sc, z));
}

int launch_dql_fold(const float2* part, int npart, float2* params, float* scale_out,
                    uint8_t* zp_out, const int* only_if, int* clear, int epoch) {
  KK_LAUNCH(dql_fold, dim3(1), dim3(kDqlFoldThreads), 0, ctx().stream, part, npart, params,
                     scale_out, zp_out, only_if, clear, epoch);
  return check_launch("dql_fold");
}

// Inputs up to kDqlSmall elements: one block of 1024 threads takes the
// (min, max), the scale and zero point and the bytes in one launch (the
// same values as the two-launch path: min and max do not depend on the
// order, and the parameters come from dql_params).  Above that one CU's
// share of the bandwidth costs more than the second launch (99840 values:
// 17 us in one block).
constexpr int64_t kDqlSmall = 16384;
constexpr int kDqlSmallThreads = 1024;

__global__ void __launch_bounds__(kDqlSmallThreads) dql_small(const float* __restrict__ x, int64_t n,
                                                              float* __restrict__ scale_out,
                                                              uint8_t* __restrict__ zp_out,
                                                              uint8_t* __restrict__ y, int vec) {
  __shared__ float smin[kDqlSmallThreads / 64], smax[kDqlSmallThreads / 64];
  __shared__ float2 pz;
  const int tid = threadIdx.x;
  const int64_t n4 = vec ? n / 4 : 0;
  float lo = INFINITY, hi = -INFINITY;
  // eight independent 16-byte loads in flight per thread (one block has to
  // cover the whole tensor: a load at a time would wait out each round trip)
  // (past the end a slot holds x[0] again, which moves neither extreme)
  constexpr int kU = 8;
  const float x0 = x[0];
  for (int64_t i0 = tid; i0 < n4; i0 += kDqlSmallThreads * kU) {
    float4 v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t i = i0 + static_cast<int64_t>(u) * kDqlSmallThreads;
      v[u] = i < n4 ? *reinterpret_cast<const float4*>(x + 4 * i)  // read again below
                    : make_float4(x0, x0, x0, x0);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      lo = fminf(lo, fminf(fminf(v[u].x, v[u].y), fminf(v[u].z, v[u].w)));
      hi = fmaxf(hi, fmaxf(fmaxf(v[u].x, v[u].y), fmaxf(v[u].z, v[u].w)));
    }
  }
  for (int64_t i = 4 * n4 + tid; i < n; i += kDqlSmallThreads) {
    lo = fminf(lo, x[i]);
    hi = fmaxf(hi, x[i]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, off, 64));
    hi = fmaxf(hi, __shfl_xor(hi, off, 64));
  }
  const int lane = tid & 63, w = tid >> 6;
  if (lane == 0) { smin[w] = lo; smax[w] = hi; }
  __syncthreads();
  if (tid == 0) {
    float fmn = smin[0], fmx = smax[0];
    for (int k = 1; k < kDqlSmallThreads / 64; ++k) {
      fmn = fminf(fmn, smin[k]);
      fmx = fmaxf(fmx, smax[k]);
    }
    pz = dql_params(fmn, fmx, scale_out, zp_out);
  }
  __syncthreads();
  const float sc = pz.x, z = pz.y;
  const KkDivisor dsc = kk_divisor(sc);
  for (int64_t i0 = tid; i0 < n4; i0 += kDqlSmallThreads * kU) {
    float4 v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t i = i0 + static_cast<int64_t>(u) * kDqlSmallThreads;
      if (i < n4) v[u] = *reinterpret_cast<const float4*>(x + 4 * i);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t i = i0 + static_cast<int64_t>(u) * kDqlSmallThreads;
      if (i < n4)
        reinterpret_cast<uint32_t*>(y)[i] = dql_bytes4(v[u], dsc, z);
    }
  }
  for (int64_t i = 4 * n4 + tid; i < n; i += kDqlSmallThreads)
    y[i] = static_cast<uint8_t>(dql_byte(x[i], sc, z));
}

// ------------------------------------------------------------------- LSTM
// One block of 1024 threads per (direction, batch row) runs the whole
// recurrence of
//   g = (xw[t] + (wb + rb)) + h @ deq(R),  deq(R) = (q - zp) * scale
// (op_lstm, ref_runtime.py:137-210; gate order i, o, f, c).
//
// The per-step product h @ (q - zp) runs on the int8 matrix cores, exactly
// in integers: h is scaled by a power of two (chosen from max|h0| for the
// first step, 2^30 after it, since |h| = |o tanh(c)| <= 1 from then on),
// rounded, and split into four signed base-256 digits, which are rows of
// the 2-of-4 sparse A operand of v_smfmac_i32_16x16x128_i8 (below); R's raw
// int8 values are the B operand and stay in registers for all steps (each
// wave owns four 16-column tiles: 64 VGPRs).  The four digit sums of a
// column recombine exactly in int64 (< 2^45), the zero point comes out
// through the integer sum of the scaled h, and the result is scaled back in
// double and rounded once to fp32.  The only approximation is the rounding
// of h to the 2^-s grid (at most 2^-31 once |h| <= 1), far below the fp32
// rounding of a 256-term dot product.
constexpr int kLstmThreads = 1024;
constexpr int kLstmMaxH = kLstmThreads / 4;
// Steps per chunk of the input projections: a chunk (4 rows of 4H floats,
// one float4 per thread) is loaded one whole chunk ahead into a double
// buffer in LDS, so the load's latency is spread over four steps, and the
// outputs of a chunk leave in one store per thread.
constexpr int kLstmChunk = 4;
typedef int lstm_v4i __attribute__((ext_vector_type(4)));
typedef int lstm_v8i __attribute__((ext_vector_type(8)));

struct LstmArgs {
  const float* xw;       // [ndir][seq * batch][4H] x @ deq(W) + (wb + rb)
  const int8_t* r;       // [ndir][H][4H]
  const void* r_scale;   // [ndir] (or 1 element)
  int r_scale_dt;
  int64_t r_scale_n;
  const void* r_zp;      // [ndir] int8 or NULL
  int r_zp_dt;
  int64_t r_zp_n;
  const float* init_h;   // [ndir][batch][H] or NULL
  const float* init_c;
  float* ys;             // [seq][ndir][batch][H]
  float* yh;             // [ndir][batch][H] or NULL
  float* yc;
  int64_t seq, batch, H, ndir;
};

// A workgroup barrier that orders LDS only: global loads (the prefetched
// input projections) and stores (the outputs) stay in flight across it,
// where __syncthreads would wait for them.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__global__ void __launch_bounds__(kLstmThreads) lstm_recurrence(LstmArgs A) {
  // R's staging area at set-up, then the double buffer of input projections
  // [2][kLstmChunk][4H] floats (both 32 KiB)
  __shared__ __align__(16) unsigned char big[32 * kLstmThreads];
  // digits of the scaled h: hd[i][p] holds digit i of the units k with
  // (k / 2) % 2 == p, at (k / 4) * 2 + k % 2 (the sparse A operand's order)
  __shared__ __align__(16) int8_t hd[4][2][kLstmMaxH / 2];
  __shared__ float gs[kLstmThreads];
  __shared__ float hring[kLstmChunk][kLstmMaxH];     // this chunk's h, for ys
  __shared__ float wmax[kLstmMaxH / 64];
  __shared__ long long wsum[kLstmMaxH / 64];
  int8_t (*rbuf)[kLstmThreads] = reinterpret_cast<int8_t (*)[kLstmThreads]>(big);
  float* xs = reinterpret_cast<float*>(big);
  const int H = static_cast<int>(A.H), G4 = 4 * H;
  const int64_t d = blockIdx.x / A.batch, b = blockIdx.x % A.batch;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar addresses
  // block-uniform: held in scalar registers (a vector register would be
  // spilled, and its reload would sit in every step)
  const float rs = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(
      int, load_as_f32(A.r_scale, A.r_scale_dt, A.r_scale_n > 1 ? d : 0))));
  long long rz =
      A.r_zp ? static_cast<long long>(load_as_i64(A.r_zp, A.r_zp_dt, A.r_zp_n > 1 ? d : 0)) : 0;
  rz = static_cast<long long>(
      (static_cast<unsigned long long>(static_cast<unsigned>(
           __builtin_amdgcn_readfirstlane(static_cast<int>(rz >> 32))))
       << 32) |
      static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<int>(rz))));
  const int8_t* R = A.r + d * static_cast<int64_t>(H) * G4;
  const float* xw = A.xw + d * A.seq * A.batch * G4;
  // B fragments: wave wv owns columns [64 wv, 64 wv + 64), four tiles of
  // 16; lane (n, g) = (lane % 16, lane / 16) holds R[ks*64 + 16g + e][col].
  // R arrives through LDS in 32-row chunks (coalesced 4-byte loads).
  lstm_v8i bf[4][2];  // [tile][k-step of 128]: the 64-row k-steps 2 kk and 2 kk + 1 side by side
#pragma unroll
  for (int chunk = 0; chunk < kLstmMaxH / 32; ++chunk) {
    __syncthreads();
    for (int idx = tid; idx < 32 * kLstmThreads / 4; idx += kLstmThreads) {
      const int row = idx / (kLstmThreads / 4), col4 = idx % (kLstmThreads / 4);
      const int k = chunk * 32 + row;
      int word = 0;
      if (k < H && 4 * col4 < G4)
        word = *reinterpret_cast<const int*>(R + static_cast<int64_t>(k) * G4 + 4 * col4);
      reinterpret_cast<int*>(rbuf[row])[col4] = word;
    }
    __syncthreads();
    const int ks = chunk / 2;                // 64-row MFMA k-step (constant once unrolled)
    const int g = lane >> 4;                 // this lane's 16 rows: ks*64 + 16g ..
    if ((g >> 1) == (chunk & 1)) {
      const int r0 = 16 * (g & 1);           // their offset inside the chunk
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const int j = (4 * wv + ct) * 16 + (lane & 15);
        int w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint32_t word = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            word |= static_cast<uint32_t>(static_cast<uint8_t>(rbuf[r0 + 4 * q + e][j])) << (8 * e);
          w[q] = static_cast<int>(word);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) bf[ct][ks >> 1][4 * (ks & 1) + q] = w[q];
      }
    }
  }
  float h = 0.0f, c = 0.0f;
  if (tid < H) {
    h = A.init_h ? A.init_h[(d * A.batch + b) * H + tid] : 0.0f;
    c = A.init_c ? A.init_c[(d * A.batch + b) * H + tid] : 0.0f;
  }
  // Chunk k holds the projections of steps 4k .. 4k+3; thread tid < 4H
  // moves float4 (tid % H) of the row of step 4k + tid / H.  Offsets from
  // the block's own rows are 32-bit (the host checks the sizes).
  const int seq = static_cast<int>(A.seq);
  const int c_t = tid < G4 ? tid : G4 - 1;  // threads past 4H repeat the last float4
  const int c_sl = c_t / H, c_c4 = c_t % H;
  // Byte offsets below 2^32 from block-uniform bases: scalar-base
  // addressing, no 64-bit address registers held across the loop.
  const char* xw_b = reinterpret_cast<const char*>(xw + b * G4);
  char* ys_b = reinterpret_cast<char*>(A.ys + (d * A.batch + b) * H);
  const uint32_t xw_row = static_cast<uint32_t>(A.batch * G4 * sizeof(float));
  const uint32_t ys_row = static_cast<uint32_t>(A.ndir * A.batch * H * sizeof(float));
  auto time_of = [&](int step) { return d == 0 ? step : seq - 1 - step; };
  // Unconditional (rows past the sequence read its last row, never used):
  // a load under a condition leaves a register copy behind it that waits
  // for the data at once.
  auto load_chunk = [&](int k) {
    int step = k * kLstmChunk + c_sl;
    step = step < seq ? step : seq - 1;
    const uint32_t off = static_cast<uint32_t>(time_of(step)) * xw_row + 16u * static_cast<uint32_t>(c_c4);
    return *reinterpret_cast<const float4*>(xw_b + off);
  };
  auto put_chunk = [&](int k, float4 v) {
    if (tid < G4) reinterpret_cast<float4*>(xs + ((k & 1) * kLstmChunk + c_sl) * G4)[c_c4] = v;
  };
  auto flush_chunk = [&](int k) {  // ys rows of chunk k from hring
    const int step = k * kLstmChunk + c_sl;
    if (tid < G4 && step < seq) {
      const uint32_t off = static_cast<uint32_t>(time_of(step)) * ys_row + 4u * static_cast<uint32_t>(c_c4);
      *reinterpret_cast<float*>(ys_b + off) = hring[c_sl][c_c4];
    }
  };
  // The first step's scale comes from max |h0| (the initial state may be
  // anything); |h * 2^shift| < 2^30.
  if (tid < kLstmMaxH) {
    const float m = wave_max(tid < H ? fabsf(h) : 0.0f);
    if (lane == 0) wmax[wv] = m;
  }
  __syncthreads();  // also ends every read of R's staging area
  int shift;
  {
    int ex = 0;
    (void)frexpf(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])), &ex);
    shift = __builtin_amdgcn_readfirstlane(30 - ex);
  }
  float4 pf = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (seq > 0) {
    put_chunk(0, load_chunk(0));
    pf = load_chunk(1);  // in flight through chunk 0
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): nothing loaded before the loop stays pending in it
  for (int step = 0; step < seq; ++step) {
    const int s = step % kLstmChunk, kc = step / kLstmChunk;
    // keep the fragments where they are (no rematerialisation across steps)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) asm volatile("" : "+v"(bf[ct][kk]));
    // (b) scale, round and split h into digits (and, with a zero point, the
    // integer sum of the scaled h).  h * 2^shift is exact in fp32 and below
    // 2^30 in magnitude, so it rounds to an int exactly.
    if (tid < kLstmMaxH) {
      const int v0 = tid < H ? static_cast<int>(rintf(ldexpf(h, shift))) : 0;
      // the balanced digits d_i in [-128, 127] with v0 = sum d_i 256^i: as
      // |v0| < 2^30, w = v0 + 0x80808080 lies in [0, 2^32) and its bytes are
      // d_i + 128 (the carries ripple in the addition), so the bytes of
      // w ^ 0x80808080 are the d_i as int8
      const uint32_t dd = (static_cast<uint32_t>(v0) + 0x80808080u) ^ 0x80808080u;
      const int hp = (tid >> 1) & 1, hpos = ((tid >> 2) << 1) | (tid & 1);
#pragma unroll
      for (int i = 0; i < 4; ++i) hd[i][hp][hpos] = static_cast<int8_t>(dd >> (8 * i));
      if (rz != 0) {
        long long sum = v0;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
        if (lane == 0) wsum[wv] = sum;
      }
    }
    lds_barrier();
    if (s == 0 && step > 0) flush_chunk(kc - 1);  // hring is rewritten after the next barrier
    const long long hsum = rz != 0 ? (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]) : 0;
    // (c) gates, on the sparse int8 matrix cores: v_smfmac_i32_16x16x128_i8
    // takes A as 2-of-4 structured (per group of four k, two values and
    // their positions) against a dense 128-k slice of R, twice the k of the
    // dense 16x16x64 for the same issue cost.  A row r (r % 8 = 2 i + p)
    // holds digit i of h at the k pairs of parity p ((k / 2) % 2 == p), the
    // other pair zero; rows 8..15 repeat 0..7.  Lane l of A (row l % 16, k
    // group l / 16 of 32) reads its sixteen values contiguously from hd[i][p];
    // R's fragments are the dense ones of k-steps 2 kk and 2 kk + 1 side by
    // side (the sparse B operand's k order).  Tile ct's lane group q then
    // holds rows 4q .. 4q+3: digits 0 and 1 (even q) or 2 and 3 (odd q), each
    // as its two parities.  Lane l takes tile l / 16, i.e. column 64 wv + l;
    // the other half of its column's digit sums comes from lane l ^ 16
    // (v_permlane16_swap), and the four recombine exactly in int64.
    lstm_v4i acc[4] = {};
    {
      const int idx = (lane & 1) ? static_cast<int>(0xEEEEEEEEu) : 0x44444444;  // positions (2, 3) / (0, 1)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const lstm_v4i a =
            *reinterpret_cast<const lstm_v4i*>(&hd[(lane >> 1) & 3][lane & 1][64 * kk + 16 * (lane >> 4)]);
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          acc[ct] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(a, bf[ct][kk], acc[ct], idx, 0, 0);
        }
      }
    }
    {
      const int q = lane >> 4;
      // two digit sums (each over both parities) recombined: |.| < 2^22 + 2^30
      int fa[4];
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) fa[ct] = (acc[ct][0] + acc[ct][1]) + ((acc[ct][2] + acc[ct][3]) << 8);
      const int own = q == 0 ? fa[0] : (q == 1 ? fa[1] : (q == 2 ? fa[2] : fa[3]));
      const int send = q == 0 ? fa[1] : (q == 1 ? fa[0] : (q == 2 ? fa[3] : fa[2]));
      // each lane keeps its own value in one of the two results and gets its
      // partner's in the other
      const auto pr = __builtin_amdgcn_permlane16_swap(send, send, false, false);
      const int recv = static_cast<int>(static_cast<unsigned>(pr[0]) + static_cast<unsigned>(pr[1]) -
                                        static_cast<unsigned>(send));
      const int lo = (q & 1) ? recv : own, hi = (q & 1) ? own : recv;
      const int j = 64 * wv + lane;
        if (j < G4) {
        const long long dot = static_cast<long long>(lo) + (static_cast<long long>(hi) << 16);
        const float hr = static_cast<float>(ldexp(static_cast<double>(dot - rz * hsum), -shift));
        const float pre = xs[((kc & 1) * kLstmChunk + s) * G4 + j] + hr * rs;  // (xw + (wb + rb)) + h @ deq(R)
        // (libm's expf and tanhf and the IEEE division: the 84-second
        // utterance's F0 curve feeds a running phase, whose end moves
        // visibly with a few-ulp change here)
        gs[j] = j < 3 * H ? 1.0f / (1.0f + expf(-pre)) : tanhf(pre);  // i, o, f: sigmoid; c: tanh
      }
    }
    lds_barrier();
    // (d) cell update of unit tid
    if (tid < H) {
      c = gs[2 * H + tid] * c + gs[tid] * gs[3 * H + tid];
      h = gs[H + tid] * tanhf(c);
      hring[s][tid] = h;
    }
    // Chunk kc + 1 goes into the buffer chunk kc - 1 used (its last reader
    // passed this step's barriers); chunk kc + 2 starts loading.
    if (s == kLstmChunk - 1) {
      put_chunk(kc + 1, pf);
      pf = load_chunk(kc + 2);
    }
    shift = 30;  // from now on |h| = |o tanh(c)| <= 1
  }
  __syncthreads();
  if (seq > 0) flush_chunk((seq - 1) / kLstmChunk);
  if (tid < H) {
    if (A.yh) A.yh[(d * A.batch + b) * H + tid] = h;
    if (A.yc) A.yc[(d * A.batch + b) * H + tid] = c;
  }
}

// ------------------------------------------------------------------- STFT
// out[b, f, k, 0/1] = sum_t (sig[b, f*step + t] * win[t]) * cos/sin(-2 pi k t / n),
// the product in fp32 and the sum in fp64 (op_stft: float32 frames @ a
// float64 basis), rounded to fp32.  Each block first builds the fp64 basis
// (the same angles, -2.0 * pi * k * t / n) and the window in LDS; a thread
// then takes one frame and all its frequencies.
__global__ void __launch_bounds__(256) stft_kernel(float* __restrict__ out,
                                                   const float* __restrict__ sig,
                                                   const void* __restrict__ win, int win_dt,
                                                   int64_t batch, int64_t slen, int64_t nframes,
                                                   int nfreq, int n, int64_t step) {
  extern __shared__ __align__(16) double stft_lds[];
  double2* basis = reinterpret_cast<double2*>(stft_lds);                // [nfreq][n] (cos, sin)
  float* w = reinterpret_cast<float*>(basis + static_cast<int64_t>(nfreq) * n);  // [n]
  for (int i = threadIdx.x; i < nfreq * n; i += blockDim.x) {
    const int k = i / n, t = i % n;
    const double ang = -2.0 * M_PI * static_cast<double>(k) * static_cast<double>(t) /
                       static_cast<double>(n);
    basis[i] = make_double2(cos(ang), sin(ang));
  }
  for (int t = threadIdx.x; t < n; t += blockDim.x) w[t] = load_as_f32(win, win_dt, t);
  __syncthreads();
  const int64_t total = batch * nframes;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t f = i % nframes, bi = i / nframes;
    const float* s = sig + bi * slen + f * step;
    float* o = out + i * nfreq * 2;
    for (int k = 0; k < nfreq; ++k) {
      const double2* bk = basis + static_cast<int64_t>(k) * n;
      double re = 0.0, im = 0.0;
      for (int t = 0; t < n; ++t) {
        const double fr = static_cast<double>(s[t] * w[t]);
        re += fr * bk[t].x;
        im += fr * bk[t].y;
      }
      o[2 * k] = static_cast<float>(re);
      o[2 * k + 1] = static_cast<float>(im);
    }
  }
}

// ----------------------------------------------------------------- Resize
// Along the last axis (op_resize, ref_runtime.py:236-256): mode 0 nearest
// (asymmetric, floor), mode 1 linear (half_pixel); positions in fp64.
__global__ void resize_kernel(float* __restrict__ out, const float* __restrict__ x, int64_t rows,
                              int64_t lin, int64_t lout, double scale, int mode) {
  const int64_t total = rows * lout;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t o = i % lout, r = i / lout;
    const float* xr = x + r * lin;
    if (mode == 0) {
      int64_t src = static_cast<int64_t>(floor(static_cast<double>(o) / scale));
      src = src < 0 ? 0 : (src > lin - 1 ? lin - 1 : src);
      out[i] = xr[src];
    } else {
      double pos = (static_cast<double>(o) + 0.5) / scale - 0.5;
      pos = pos < 0.0 ? 0.0 : (pos > static_cast<double>(lin - 1) ? static_cast<double>(lin - 1) : pos);
      const int64_t i0 = static_cast<int64_t>(floor(pos));
      const int64_t i1 = i0 + 1 > lin - 1 ? lin - 1 : i0 + 1;
      const float frac = static_cast<float>(pos - static_cast<double>(i0));
      out[i] = xr[i0] * (1.0f - frac) + xr[i1] * frac;
    }
  }
}

// -------------------------------------------------------------------- Pad
// numpy.pad semantics (op_pad): mode 0 constant, 1 reflect (mirror without
// repeating the edge), 2 edge.
struct PadArgs {
  int rank;
  int64_t in_dims[KK_MAX_RANK], out_dims[KK_MAX_RANK], begin[KK_MAX_RANK];
  int64_t in_st[KK_MAX_RANK];
  int mode;
  float value;
  int64_t n;
};

__device__ __forceinline__ int64_t reflect_index(int64_t i, int64_t dim) {
  if (dim == 1) return 0;
  const int64_t period = 2 * (dim - 1);
  int64_t m = i % period;
  if (m < 0) m += period;
  return m < dim ? m : period - m;
}

__global__ void pad_kernel(float* __restrict__ out, const float* __restrict__ x, PadArgs P) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < P.n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t rem = i, off = 0;
    bool inside = true;
    for (int d = P.rank - 1; d >= 0; --d) {
      const int64_t o = rem % P.out_dims[d];
      rem /= P.out_dims[d];
      int64_t s = o - P.begin[d];
      const int64_t dim = P.in_dims[d];
      if (s < 0 || s >= dim) {
        if (P.mode == 0) inside = false;
        else if (P.mode == 1) s = reflect_index(s, dim);
        else s = s < 0 ? 0 : dim - 1;
      }
      off += s * P.in_st[d];
    }
    out[i] = inside ? x[off] : P.value;
  }
}

// Pad with one block row per output row (all axes but the last): the row's
// source offset is worked out once, the last axis walked contiguously.
__global__ void pad_rows_kernel(float* __restrict__ out, const float* __restrict__ x, PadArgs P,
                                int64_t rows) {
  const int last = P.rank - 1;
  const int64_t lout = P.out_dims[last], dim = P.in_dims[last], b = P.begin[last];
  const int64_t st = P.in_st[last];
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    int64_t rem = r, off = 0;
    bool inside = true;
    for (int d = last - 1; d >= 0; --d) {
      const int64_t o = rem % P.out_dims[d];
      rem /= P.out_dims[d];
      int64_t s = o - P.begin[d];
      const int64_t dd = P.in_dims[d];
      if (s < 0 || s >= dd) {
        if (P.mode == 0) inside = false;
        else if (P.mode == 1) s = reflect_index(s, dd);
        else s = s < 0 ? 0 : dd - 1;
      }
      off += s * P.in_st[d];
    }
    float* orow = out + r * lout;
    for (int64_t o = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; o < lout;
         o += static_cast<int64_t>(gridDim.x) * blockDim.x) {
      int64_t s = o - b;
      bool in = inside;
      if (s < 0 || s >= dim) {
        if (P.mode == 0) in = false;
        else if (P.mode == 1) s = reflect_index(s, dim);
        else s = s < 0 ? 0 : dim - 1;
      }
      orow[o] = in ? x[off + s * st] : P.value;
    }
  }
}

// ----------------------------------------------------------------- CumSum
// One thread per line, a sequential running sum in the input's type (numpy
// cumsum accumulates in order, so fp32 results match bit for bit).
// Lines of at most kCumsumLds fp32 values: a block per line stages it in
// LDS, one thread runs the sum there (its reads do not wait on the chain
// of additions, as global loads would), the block writes the line back.
constexpr int kCumsumLds = 16384;

__global__ void __launch_bounds__(256) cumsum_lds_kernel(float* __restrict__ out,
                                                         const float* __restrict__ x,
                                                         int64_t dim, int64_t inner) {
  __shared__ __align__(16) float buf[kCumsumLds];
  const int64_t line = blockIdx.x;
  const int64_t o = line / inner, in = line % inner;
  const float* xs = x + o * dim * inner + in;
  float* os = out + o * dim * inner + in;
  const int n = static_cast<int>(dim);
  for (int d = threadIdx.x; d < n; d += blockDim.x) buf[d] = xs[d * inner];
  __syncthreads();
  if (threadIdx.x == 0) {
    float acc = 0.0f;
    int d = 0;
    for (; d + 4 <= n; d += 4) {
      float4 v = *reinterpret_cast<const float4*>(buf + d);
      acc = acc + v.x; v.x = acc;
      acc = acc + v.y; v.y = acc;
      acc = acc + v.z; v.z = acc;
      acc = acc + v.w; v.w = acc;
      *reinterpret_cast<float4*>(buf + d) = v;
    }
    for (; d < n; ++d) {
      acc = acc + buf[d];
      buf[d] = acc;
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < n; d += blockDim.x) os[d * inner] = buf[d];
}

template <typename T>
__global__ void cumsum_kernel(T* __restrict__ out, const T* __restrict__ x, int64_t outer,
                              int64_t dim, int64_t inner) {
  const int64_t lines = outer * inner;
  for (int64_t l = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; l < lines;
       l += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t o = l / inner, in = l % inner;
    const T* xs = x + o * dim * inner + in;
    T* os = out + o * dim * inner + in;
    T acc = 0;
    for (int64_t d = 0; d < dim; ++d) {
      acc = acc + xs[d * inner];
      os[d * inner] = acc;
    }
  }
}

// -------------------------------------------------------------- ScatterND
// out[idx[i]] = updates[i] for slices of `inner` elements; the host has
// already removed duplicate indices (keeping the last, as the reference's
// sequential loop does), so no two threads write one element.
__global__ void scatter_kernel(uint8_t* __restrict__ out, const uint8_t* __restrict__ upd,
                               const int64_t* __restrict__ offsets, int64_t nidx, int64_t inner,
                               int elem) {
  const int64_t total = nidx * inner;
  for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i = t / inner, e = t % inner;
    const int64_t dst = (offsets[i] + e) * elem, src = t * elem;
    for (int k = 0; k < elem; ++k) out[dst + k] = upd[src + k];
  }
}

static unsigned grid1d(int64_t n) {
  return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 256), 1 << 16)));
}

static int f32_contig(const kk_tensor* t, const char* name) {
  KK_TRY(check_tensor(t, name));
  if (t->dtype != KK_F32) return set_error(KK_E_ARG, "%s must be fp32", name);
  if (!is_contiguous(t)) return set_error(KK_E_ARG, "%s must be contiguous", name);
  return KK_OK;
}

}  // namespace kk

using namespace kk;

extern "C" {

int kk_dynamic_quantize_linear(const kk_tensor* y, const kk_tensor* scale, const kk_tensor* zp,
                               const kk_tensor* x) {
  KK_TRY(require_ready());
  KK_TRY(f32_contig(x, "x"));
  KK_TRY(check_tensor(y, "y"));
  KK_TRY(check_tensor(scale, "scale"));
  KK_TRY(check_tensor(zp, "zp"));
  if (y->dtype != KK_U8 || !is_contiguous(y) || numel(y) != numel(x))
    return set_error(KK_E_ARG, "kk_dynamic_quantize_linear: y must be contiguous uint8 like x");
  if (scale->dtype != KK_F32 || numel(scale) != 1 || zp->dtype != KK_U8 || numel(zp) != 1)
    return set_error(KK_E_ARG, "kk_dynamic_quantize_linear: scale is one fp32, zp one uint8");
  const int64_t n = numel(x);
  if (n == 0) return set_error(KK_E_ARG, "kk_dynamic_quantize_linear: empty input");
  const int nblk = static_cast<int>(std::min<int64_t>(kDqlBlocks, ceil_div(n, 4096)));
  const int vec = (reinterpret_cast<uintptr_t>(x->data) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(y->data) % 4 == 0) ? 1 : 0;
  if (n <= kDqlSmall) {
    KK_LAUNCH(dql_small, dim3(1), dim3(kDqlSmallThreads), 0, ctx().stream,
                       static_cast<const float*>(x->data), n, static_cast<float*>(scale->data),
                       static_cast<uint8_t*>(zp->data), static_cast<uint8_t*>(y->data), vec);
    return check_launch("dql_small");
  }
  // the partials in the context's scratch
  static_assert(sizeof(float2) * kDqlBlocks <= kScratchBytes, "DQL partials");
  float2* pp = static_cast<float2*>(ctx().scratch);
  KK_LAUNCH(dql_minmax_part, dim3(nblk), dim3(256), 0, ctx().stream,
                     static_cast<const float*>(x->data), n, pp, vec);
  KK_TRY(check_launch("dql_minmax_part"));
  const unsigned g = static_cast<unsigned>(std::min<int64_t>(ceil_div(n, 1024), 4096));
  KK_LAUNCH(dql_quantize_fold, dim3(g), dim3(256), 0, ctx().stream,
                     static_cast<const float*>(x->data), n, static_cast<const float2*>(pp), nblk,
                     static_cast<float*>(scale->data), static_cast<uint8_t*>(zp->data),
                     static_cast<uint8_t*>(y->data), vec);
  return check_launch("dql_quantize_fold");
}

int kk_lstm(const kk_tensor* ys, const kk_tensor* yh, const kk_tensor* yc, const kk_tensor* x,
            const kk_tensor* w, const kk_tensor* r, const kk_tensor* b, const kk_tensor* init_h,
            const kk_tensor* init_c, const kk_tensor* w_scale, const kk_tensor* w_zp,
            const kk_tensor* r_scale, const kk_tensor* r_zp, int hidden_size, int bidirectional) {
  KK_TRY(require_ready());
  KK_TRY(f32_contig(x, "x"));
  KK_TRY(f32_contig(ys, "ys"));
  KK_TRY(check_tensor(w, "w"));
  KK_TRY(check_tensor(r, "r"));
  KK_TRY(check_tensor(w_scale, "w_scale"));
  KK_TRY(check_tensor(r_scale, "r_scale"));
  const int64_t H = hidden_size, ndir = bidirectional ? 2 : 1;
  if (x->rank != 3) return set_error(KK_E_ARG, "kk_lstm: x must be [seq, batch, input]");
  const int64_t seq = x->shape[0], batch = x->shape[1], in = x->shape[2];
  if (w->dtype != KK_I8 || r->dtype != KK_I8 || !is_contiguous(w) || !is_contiguous(r))
    return set_error(KK_E_ARG, "kk_lstm: W and R must be contiguous int8");
  if (w->rank != 3 || w->shape[0] != ndir || w->shape[1] != in || w->shape[2] != 4 * H)
    return set_error(KK_E_ARG, "kk_lstm: W must be [dir, input, 4H]");
  if (r->rank != 3 || r->shape[0] != ndir || r->shape[1] != H || r->shape[2] != 4 * H)
    return set_error(KK_E_ARG, "kk_lstm: R must be [dir, H, 4H]");
  if (H < 1 || H > kLstmMaxH)
    return set_error(KK_E_UNSUPPORTED, "kk_lstm: hidden size %lld (1..%d)", (long long)H, kLstmMaxH);
  if (numel(ys) != seq * ndir * batch * H) return set_error(KK_E_ARG, "kk_lstm: ys shape");
  if (seq * ndir * batch * 4 * H >= (int64_t{1} << 30))  // the kernel's 32-bit byte offsets
    return set_error(KK_E_UNSUPPORTED, "kk_lstm: seq * dir * batch * 4H must stay below 2^30");
  const int64_t nws = numel(w_scale), nrs = numel(r_scale);
  if ((nws != 1 && nws != ndir) || (nrs != 1 && nrs != ndir))
    return set_error(KK_E_ARG, "kk_lstm: scales need 1 or dir elements");
  if (b) {
    KK_TRY(f32_contig(b, "b"));
    if (numel(b) != ndir * 8 * H) return set_error(KK_E_ARG, "kk_lstm: B must be [dir, 8H]");
  }
  for (const kk_tensor* t : {init_h, init_c, yh, yc})
    if (t) {
      KK_TRY(f32_contig(t, "state"));
      if (numel(t) != ndir * batch * H) return set_error(KK_E_ARG, "kk_lstm: state shape");
    }
  // Input projections xw[d] = x @ deq(W[d]) + (wb[d] + rb[d]) on the MFMA
  // GEMM and two elementwise adds (the biases summed first, as op_lstm does).
  void* xw = nullptr;
  const int64_t xw_n = ndir * seq * batch * 4 * H;
  const int64_t xw_bytes = ((sizeof(float) * std::max<int64_t>(xw_n, 1) + 255) / 256) * 256;
  KK_TRY(kk_alloc(static_cast<size_t>(xw_bytes + sizeof(float) * 4 * H), &xw));
  float* bsum = reinterpret_cast<float*>(static_cast<char*>(xw) + xw_bytes);
  int rc = KK_OK;
  for (int64_t d = 0; d < ndir && rc == KK_OK && seq * batch > 0; ++d) {
    kk_tensor a{}, wd{}, o{}, sc{}, zpt{};
    a.data = x->data; a.dtype = KK_F32; a.rank = 2;
    a.shape[0] = seq * batch; a.shape[1] = in; a.strides[0] = in; a.strides[1] = 1;
    wd.data = static_cast<int8_t*>(w->data) + d * in * 4 * H; wd.dtype = KK_I8; wd.rank = 2;
    wd.shape[0] = in; wd.shape[1] = 4 * H; wd.strides[0] = 4 * H; wd.strides[1] = 1;
    o.data = static_cast<float*>(xw) + d * seq * batch * 4 * H; o.dtype = KK_F32; o.rank = 2;
    o.shape[0] = seq * batch; o.shape[1] = 4 * H; o.strides[0] = 4 * H; o.strides[1] = 1;
    sc.data = static_cast<char*>(w_scale->data) + (nws > 1 ? d * dtype_size(w_scale->dtype) : 0);
    sc.dtype = w_scale->dtype; sc.rank = 0;
    const kk_tensor* zptr = nullptr;
    if (w_zp) {
      zpt.data = static_cast<char*>(w_zp->data) + (numel(w_zp) > 1 ? d * dtype_size(w_zp->dtype) : 0);
      zpt.dtype = w_zp->dtype; zpt.rank = 0;
      zptr = &zpt;
    }
    // the recurrence amplifies the projection's rounding: keep numpy's
    // (each dequantised weight rounded to fp32, exact fp32 products)
    rc = gemm(&o, &a, &wd, &sc, zptr, 1.0f, true);
    if (rc == KK_OK && b) {
      kk_tensor wb{}, rb{}, bs{};
      for (kk_tensor* t : {&wb, &rb, &bs}) {
        t->dtype = KK_F32; t->rank = 2; t->shape[0] = 1; t->shape[1] = 4 * H;
        t->strides[0] = 4 * H; t->strides[1] = 1;
      }
      wb.data = static_cast<float*>(b->data) + d * 8 * H;
      rb.data = static_cast<float*>(b->data) + d * 8 * H + 4 * H;
      bs.data = bsum;
      rc = kk_binary(KK_OP_ADD, &bs, &wb, &rb);
      if (rc == KK_OK) {
        bs.shape[0] = 1;
        bs.strides[0] = 0;  // broadcast over the rows of xw[d]
        bs.shape[0] = seq * batch;
        rc = kk_binary(KK_OP_ADD, &o, &o, &bs);
      }
    }
  }
  if (rc == KK_OK) {
    LstmArgs A{};
    A.xw = static_cast<const float*>(xw);
    A.r = static_cast<const int8_t*>(r->data);
    A.r_scale = r_scale->data; A.r_scale_dt = r_scale->dtype; A.r_scale_n = nrs;
    if (r_zp) { A.r_zp = r_zp->data; A.r_zp_dt = r_zp->dtype; A.r_zp_n = numel(r_zp); }
    A.init_h = init_h ? static_cast<const float*>(init_h->data) : nullptr;
    A.init_c = init_c ? static_cast<const float*>(init_c->data) : nullptr;
    A.ys = static_cast<float*>(ys->data);
    A.yh = yh ? static_cast<float*>(yh->data) : nullptr;
    A.yc = yc ? static_cast<float*>(yc->data) : nullptr;
    A.seq = seq; A.batch = batch; A.H = H; A.ndir = ndir;
    KK_LAUNCH(lstm_recurrence, dim3(static_cast<unsigned>(ndir * batch)),
                       dim3(kLstmThreads), 0, ctx().stream, A);
    rc = check_launch("lstm_recurrence");
  }
  kk_free(xw);
  return rc;
}

int kk_stft(const kk_tensor* out, const kk_tensor* signal, const kk_tensor* window,
            int64_t frame_step, int64_t frame_length, int onesided) {
  KK_TRY(require_ready());
  KK_TRY(f32_contig(signal, "signal"));
  KK_TRY(f32_contig(out, "out"));
  KK_TRY(check_tensor(window, "window"));
  if (!is_float(window->dtype) || numel(window) != frame_length)
    return set_error(KK_E_ARG, "kk_stft: window must hold frame_length floats");
  if (frame_step < 1 || frame_length < 1) return set_error(KK_E_ARG, "kk_stft: bad frame sizes");
  const int64_t batch = signal->shape[0];
  const int64_t slen = numel(signal) / std::max<int64_t>(batch, 1);
  const int64_t nframes = slen >= frame_length ? (slen - frame_length) / frame_step + 1 : 0;
  const int64_t nfreq = onesided ? frame_length / 2 + 1 : frame_length;
  if (numel(out) != batch * nframes * nfreq * 2)
    return set_error(KK_E_ARG, "kk_stft: out must be [batch, %lld, %lld, 2]", (long long)nframes,
                     (long long)nfreq);
  const int64_t total = batch * nframes;
  if (!total || !nfreq) return KK_OK;
  const size_t lds = sizeof(double) * 2 * static_cast<size_t>(nfreq * frame_length) +
                     sizeof(float) * static_cast<size_t>(frame_length);
  if (lds > 64 * 1024)
    return set_error(KK_E_UNSUPPORTED, "kk_stft: frame_length %lld too long (basis > 64 KB)",
                     (long long)frame_length);
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(ceil_div(total, 256), 1024));
  KK_LAUNCH(stft_kernel, dim3(blocks), dim3(256), lds, ctx().stream,
                     static_cast<float*>(out->data), static_cast<const float*>(signal->data),
                     window->data, window->dtype, batch, slen, nframes, static_cast<int>(nfreq),
                     static_cast<int>(frame_length), frame_step);
  return check_launch("stft_kernel");
}

int kk_resize(const kk_tensor* out, const kk_tensor* x, int mode, double scale) {
  KK_TRY(require_ready());
  KK_TRY(f32_contig(x, "x"));
  KK_TRY(f32_contig(out, "out"));
  if (mode != 0 && mode != 1) return set_error(KK_E_ARG, "kk_resize: mode 0 or 1");
  if (x->rank < 1 || out->rank != x->rank) return set_error(KK_E_ARG, "kk_resize: ranks");
  const int64_t lin = x->shape[x->rank - 1], lout = out->shape[out->rank - 1];
  if (lout != static_cast<int64_t>(std::floor(lin * scale)))
    return set_error(KK_E_ARG, "kk_resize: out length must be floor(L * scale)");
  for (int i = 0; i < x->rank - 1; ++i)
    if (x->shape[i] != out->shape[i]) return set_error(KK_E_ARG, "kk_resize: leading axes differ");
  const int64_t rows = lin ? numel(x) / lin : 0;
  if (!rows || !lout) return KK_OK;
  KK_LAUNCH(resize_kernel, dim3(grid1d(rows * lout)), dim3(256), 0, ctx().stream,
                     static_cast<float*>(out->data), static_cast<const float*>(x->data), rows, lin,
                     lout, scale, mode);
  return check_launch("resize_kernel");
}

int kk_pad(const kk_tensor* out, const kk_tensor* x, const int64_t* pads, int mode, float value) {
  KK_TRY(require_ready());
  KK_TRY(check_tensor(x, "x"));
  KK_TRY(f32_contig(out, "out"));
  if (x->dtype != KK_F32) return set_error(KK_E_ARG, "kk_pad: x must be fp32");
  if (!pads) return set_error(KK_E_ARG, "kk_pad: pads is NULL");
  if (mode < 0 || mode > 2) return set_error(KK_E_ARG, "kk_pad: mode 0/1/2");
  PadArgs P{};
  P.rank = x->rank;
  P.mode = mode;
  P.value = value;
  P.n = 1;
  for (int d = 0; d < x->rank; ++d) {
    const int64_t b0 = pads[d], b1 = pads[d + x->rank];
    if (b0 < 0 || b1 < 0) return set_error(KK_E_UNSUPPORTED, "kk_pad: negative pads");
    if (mode != 0 && (b0 || b1) && x->shape[d] == 0)
      return set_error(KK_E_ARG, "kk_pad: cannot reflect or extend an empty axis");
    P.in_dims[d] = x->shape[d];
    P.in_st[d] = x->strides[d];
    P.begin[d] = b0;
    P.out_dims[d] = x->shape[d] + b0 + b1;
    if (out->shape[d] != P.out_dims[d]) return set_error(KK_E_ARG, "kk_pad: out shape");
    P.n *= P.out_dims[d];
  }
  if (out->rank != x->rank) return set_error(KK_E_ARG, "kk_pad: out rank");
  if (!P.n) return KK_OK;
  const int64_t lout = P.out_dims[P.rank - 1];
  if (lout >= 1024) {
    const int64_t rows = P.n / lout;
    const dim3 grid(static_cast<unsigned>(std::min<int64_t>(ceil_div(lout, 256 * 4), 1 << 16)),
                    static_cast<unsigned>(std::min<int64_t>(rows, 65535)));
    KK_LAUNCH(pad_rows_kernel, grid, dim3(256), 0, ctx().stream,
                       static_cast<float*>(out->data), static_cast<const float*>(x->data), P, rows);
    return check_launch("pad_rows_kernel");
  }
  KK_LAUNCH(pad_kernel, dim3(grid1d(P.n)), dim3(256), 0, ctx().stream,
                     static_cast<float*>(out->data), static_cast<const float*>(x->data), P);
  return check_launch("pad_kernel");
}

int kk_cumsum(const kk_tensor* out, const kk_tensor* x, int axis) {
  KK_TRY(require_ready());
  KK_TRY(check_tensor(x, "x"));
  KK_TRY(check_tensor(out, "out"));
  if (!is_contiguous(x) || !is_contiguous(out) || x->dtype != out->dtype || numel(x) != numel(out))
    return set_error(KK_E_ARG, "kk_cumsum: contiguous x and out of one dtype and size");
  if (x->rank == 0) return set_error(KK_E_ARG, "kk_cumsum: scalar input");
  if (axis < 0) axis += x->rank;
  if (axis < 0 || axis >= x->rank) return set_error(KK_E_ARG, "kk_cumsum: axis");
  int64_t outer = 1, inner = 1;
  for (int i = 0; i < axis; ++i) outer *= x->shape[i];
  for (int i = axis + 1; i < x->rank; ++i) inner *= x->shape[i];
  const int64_t dim = x->shape[axis];
  if (!numel(x)) return KK_OK;
  const dim3 g(grid1d(outer * inner));
  if (x->dtype == KK_F32 && dim <= kCumsumLds && outer * inner <= 0x7fffffff) {
    KK_LAUNCH(cumsum_lds_kernel, dim3(static_cast<unsigned>(outer * inner)), dim3(256), 0,
                       ctx().stream, static_cast<float*>(out->data), static_cast<const float*>(x->data),
                       dim, inner);
    return check_launch("cumsum_lds_kernel");
  }
  switch (x->dtype) {
    case KK_F32:
      KK_LAUNCH(cumsum_kernel<float>, g, dim3(256), 0, ctx().stream,
                         static_cast<float*>(out->data), static_cast<const float*>(x->data), outer,
                         dim, inner);
      break;
    case KK_I64:
      KK_LAUNCH(cumsum_kernel<int64_t>, g, dim3(256), 0, ctx().stream,
                         static_cast<int64_t*>(out->data), static_cast<const int64_t*>(x->data),
                         outer, dim, inner);
      break;
    case KK_I32:
      KK_LAUNCH(cumsum_kernel<int32_t>, g, dim3(256), 0, ctx().stream,
                         static_cast<int32_t*>(out->data), static_cast<const int32_t*>(x->data),
                         outer, dim, inner);
      break;
    default:
      return set_error(KK_E_UNSUPPORTED, "kk_cumsum: dtype %d", x->dtype);
  }
  return check_launch("cumsum_kernel");
}

int kk_scatter_nd(const kk_tensor* out, const kk_tensor* updates, const int64_t* offsets,
                  int64_t nidx, int64_t inner) {
  KK_TRY(require_ready());
  KK_TRY(check_tensor(out, "out"));
  KK_TRY(check_tensor(updates, "updates"));
  if (!is_contiguous(out) || !is_contiguous(updates) || updates->dtype != out->dtype)
    return set_error(KK_E_ARG, "kk_scatter_nd: contiguous out and updates of one dtype");
  if (nidx < 0 || inner < 0 || (nidx && !offsets))
    return set_error(KK_E_ARG, "kk_scatter_nd: bad offsets");
  if (numel(updates) != nidx * inner) return set_error(KK_E_ARG, "kk_scatter_nd: updates size");
  const int64_t n = numel(out);
  for (int64_t i = 0; i < nidx; ++i)
    if (offsets[i] < 0 || offsets[i] + inner > n)
      return set_error(KK_E_ARG, "kk_scatter_nd: offset %lld out of range", (long long)offsets[i]);
  if (!nidx || !inner) return KK_OK;
  void* dev = nullptr;
  KK_TRY(kk_alloc(sizeof(int64_t) * nidx, &dev));
  int rc = kk_upload(dev, offsets, sizeof(int64_t) * nidx);
  if (rc == KK_OK) {
    KK_LAUNCH(scatter_kernel, dim3(grid1d(nidx * inner)), dim3(256), 0, ctx().stream,
                       static_cast<uint8_t*>(out->data), static_cast<const uint8_t*>(updates->data),
                       static_cast<const int64_t*>(dev), nidx, inner, dtype_size(out->dtype));
    rc = check_launch("scatter_kernel");
  }
  kk_free(dev);
  return rc;
}

}  // extern "C"
