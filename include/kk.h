/*
 * kk.h -- C ABI of libkk, the MI355X (gfx950) tensor-op layer for the
 * quantized Kokoro-82M graph.
 *
 * libkk replaces the numpy op layer `RefRuntime.dispatch`
 * (tools/ref_runtime.py:428-668) and the GLSL twin of that layer
 * (addons/best-tts/runtime/executor.gd:733-843 over runtime/gpu.gd:233-249).
 * A host-side `dispatch(op, node_input, node_output, attrs, env)` with the
 * reference's signature calls these entry points through ctypes.
 *
 * Conventions
 *  - Every entry point returns 0 on success and a negative KK_E* code on
 *    failure; it never aborts.  kk_last_error() describes the last failure of
 *    the calling thread.
 *  - All work is enqueued on the library's one HIP stream, in call order.
 *    kk_download() and kk_sync() wait for it; nothing else blocks.
 *  - Tensors are described by kk_tensor: a device pointer to element
 *    [0,...,0], a dtype code and up to KK_MAX_RANK extents and element
 *    strides.  A stride of 0 marks a broadcast axis.  Shapes follow numpy:
 *    inputs of an elementwise op are right-aligned against the output shape.
 *  - Arithmetic is fp32 whatever the storage type (fp16 is storage only,
 *    tools/NOTES.md:44-59).
 */
#ifndef KK_H
#define KK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KK_MAX_RANK 8

/* dtype codes: the KPK1 codes of tools/kpk_runtime.py:21-24
 * (also tools/pack_model.py:38-44). */
enum {
  KK_F32 = 0, KK_I8 = 1, KK_U8 = 2, KK_I32 = 3, KK_I64 = 4, KK_BOOL = 5,
  KK_F16 = 6
};

/* status codes */
enum {
  KK_OK = 0,
  KK_E_ARG = -1,      /* invalid argument, shape or dtype */
  KK_E_HIP = -2,      /* a HIP runtime call failed */
  KK_E_NOMEM = -3,    /* device allocation failed */
  KK_E_STATE = -4,    /* library not initialised, or double free */
  KK_E_UNSUPPORTED = -5
};

typedef struct kk_tensor {
  void*   data;                     /* device address of element [0,..,0] */
  int32_t dtype;                    /* KK_F32 .. KK_F16 */
  int32_t rank;                     /* 0 .. KK_MAX_RANK */
  int64_t shape[KK_MAX_RANK];
  int64_t strides[KK_MAX_RANK];     /* in elements; 0 = broadcast */
} kk_tensor;

/* ---------------------------------------------------------------- lifecycle
 * Replaces KokoroGPU.initialize/cleanup/submit_and_wait
 * (addons/best-tts/runtime/gpu.gd:35-41, 266-268): one device, one stream. */
int         kk_init(int device);
int         kk_shutdown(void);
int         kk_sync(void);
const char* kk_last_error(void);
int         kk_device_count(int* count);

/* --------------------------------------------------------------- buffer pool
 * Replaces the executor's pool: _bucket/_alloc/_release/trim_memory
 * (addons/best-tts/runtime/executor.gd:206-268, 400-425) and numpy's
 * per-op allocation (tools/ref_runtime.py:668).  Sizes are rounded up to a
 * bucket that keeps four significant bits (256 B minimum); freed buffers are
 * kept per bucket and handed out again; a second free of one buffer is
 * rejected with KK_E_STATE. */
int kk_alloc(size_t bytes, void** dptr);
int kk_free(void* dptr);
int kk_pool_stats(size_t* live_bytes, size_t* pooled_bytes,
                  size_t* peak_live_bytes);
int kk_pool_trim(size_t budget_bytes);
/* Host <-> device copies (gpu.gd:88-103 create_buffer / read_f32).
 * kk_upload returns as soon as the source may be reused (its bytes are
 * captured in kernel arguments or a pinned staging ring) without waiting for
 * the stream; the device copy runs in stream order before any later op.
 * Uploads above 16 MB complete before returning.  kk_download returns after
 * the copy (and all earlier work on the stream) has completed. */
int kk_upload(void* dst_device, const void* src_host, size_t bytes);
int kk_download(void* dst_host, const void* src_device, size_t bytes);

/* ------------------------------------------------------ elementwise family
 * Broadcast elementwise ops, the Add/Sub/Mul/Div/Pow/... branches of
 * tools/ref_runtime.py:446-503 and the GLSL twin elementwise.glsl:43-160
 * with its broadcast indexer runtime/ops.gd:45-129.  `out` may be strided
 * (writes into a view) but must not broadcast. */
enum {
  KK_OP_ADD = 0, KK_OP_SUB = 1, KK_OP_MUL = 2, KK_OP_DIV = 3, KK_OP_POW = 4,
  KK_OP_SQRT = 5, KK_OP_EXP = 6, KK_OP_SIN = 7, KK_OP_COS = 8,
  KK_OP_ATAN = 9, KK_OP_TANH = 10, KK_OP_SIGMOID = 11, KK_OP_FLOOR = 12,
  KK_OP_ROUND = 13, KK_OP_LEAKYRELU = 14, KK_OP_EQUAL = 16,
  KK_OP_GREATER = 17, KK_OP_LESS = 18, KK_OP_GEQ = 19, KK_OP_AND = 20,
  KK_OP_NEG = 25, KK_OP_ABS = 26, KK_OP_LOG = 27, KK_OP_MIN = 28,
  KK_OP_MAX = 29, KK_OP_ERF = 30, KK_OP_IDENTITY = 24
};

/* Add/Sub/Mul/Div/Pow/Min/Max and comparisons: ref_runtime.py:446-457,
 * 492-501.  Float inputs (f32/f16) compute in fp32; two integer inputs
 * compute in int64 with Div as floor division (:453-455). */
int kk_binary(int op, const kk_tensor* out, const kk_tensor* a,
              const kk_tensor* b);
/* Sqrt/Exp/Sin/Cos/Atan/Tanh/Sigmoid/Floor/Round/LeakyRelu/Neg/Abs/Log/Erf:
 * ref_runtime.py:458-479, 487-489.  `alpha` is LeakyRelu's slope. */
int kk_unary(int op, const kk_tensor* out, const kk_tensor* x, float alpha);
/* Where(cond, x, y): ref_runtime.py:502-503. */
int kk_where(const kk_tensor* out, const kk_tensor* cond, const kk_tensor* x,
             const kk_tensor* y);
/* Clip(x, lo, hi), lo/hi may be NULL: ref_runtime.py:480-486. */
int kk_clip(const kk_tensor* out, const kk_tensor* x, const kk_tensor* lo,
            const kk_tensor* hi);
/* Fused snake activation y = x + r * sin(alpha*x)^2, the five-node chain
 * Mul -> Sin -> Pow(2) -> Mul(recip) -> Add of the graph (kpk #2853-2857,
 * built from ref_runtime.py:446-463).  If `recip` is NULL, r = 1/alpha in
 * fp32.  alpha/recip broadcast like any operand (normally [1,C,1]). */
int kk_snake(const kk_tensor* out, const kk_tensor* x, const kk_tensor* alpha,
             const kk_tensor* recip);
/* FastGelu(x, bias): ref_runtime.py:288-293; bias may be NULL. */
int kk_fast_gelu(const kk_tensor* out, const kk_tensor* x,
                 const kk_tensor* bias);
/* DequantizeLinear: (q - zp) * scale in fp32, ref_runtime.py:631-636;
 * zp may be NULL. */
int kk_dequantize(const kk_tensor* out, const kk_tensor* q,
                  const kk_tensor* scale, const kk_tensor* zp);

/* ------------------------------------------------------------ data movement
 * Strided copy with dtype conversion.  Serves Cast (ref_runtime.py:572-578:
 * fp16 targets store fp32, float->int truncates), Transpose/Expand/Concat
 * materialisation (:517-518, :531-535, :553-555) and the copy.glsl twin.
 * `x` may broadcast against `out`. */
int kk_copy(const kk_tensor* out, const kk_tensor* x);
/* ConstantOfShape / zero fill (ref_runtime.py:556-559). */
int kk_fill(const kk_tensor* out, double value);
/* Gather: np.take(data, indices, axis) (ref_runtime.py:550-552), the GLSL
 * twin gather.glsl.  Negative indices count from the end; indices outside
 * [-dim, dim) are clamped on the device (the host checks host-side ones). */
int kk_gather(const kk_tensor* out, const kk_tensor* data,
              const kk_tensor* indices, int axis);

/* ------------------------------------------------------------- reductions
 * ReduceMean/ReduceSum/ReduceMax over the axes in `axes_mask` (bit i =
 * axis i of x): ref_runtime.py:589-598.  `out` holds the kept axes in
 * order (keepdims is a view question for the caller). */
enum { KK_REDUCE_SUM = 0, KK_REDUCE_MEAN = 1, KK_REDUCE_MAX = 2 };
int kk_reduce(int op, const kk_tensor* out, const kk_tensor* x,
              uint32_t axes_mask);
/* Instance norm over the last axis of x [N,C,T] with the AdaIN affine:
 *   y = (x - mean_T) / sqrt(var_T + eps) * (1 + gamma[c]) + beta[c]
 * (graph kpk #2844-2852: ReduceMean, Sub, Mul, ReduceMean, Add, Sqrt, Div,
 * Mul(1+gamma), Add(beta)).  gamma_beta is h = [gamma | beta] of 2C floats
 * (the Split of kpk #80 -> #138); NULL gives gamma = beta = 0. */
int kk_instance_norm_affine(const kk_tensor* out, const kk_tensor* x,
                            const kk_tensor* gamma_beta, float eps);
/* The graph's InstanceNorm chain fused: ReduceMean -> Sub -> Mul(d, d) ->
 * ReduceMean -> Add(eps) -> Sqrt -> Div -> Mul(scale) -> Add(shift), and an
 * optional LeakyRelu(alpha) after it (ref_runtime.py:589-598 ReduceMean,
 * :446-455 Sub/Mul/Add/Div, :458-459 Sqrt, :476-479 LeakyRelu):
 *   y = (x - mean_T) / sqrt(var_T + eps) * scale[c] + shift[c]
 * over the last axis of x [N, C, T]; scale/shift hold C floats or are NULL
 * (factor 1 / offset 0).  Rows longer than 16384 are split across blocks. */
int kk_instance_norm_scale_shift(const kk_tensor* out, const kk_tensor* x,
                                 const kk_tensor* scale, const kk_tensor* shift, float eps,
                                 int leaky, float alpha);
/* The same chain followed by the graph's snake chain on its output,
 * Mul(alpha, y) -> Sin -> Pow(2) -> Mul(recip) -> Add(y) (ref_runtime.py
 * :446-463; kk_snake): z = y + recip[c] * sin(alpha[c] * y)^2, one pass
 * instead of two.  alpha and recip hold C floats. */
int kk_instance_norm_scale_shift_snake(const kk_tensor* out, const kk_tensor* x,
                                       const kk_tensor* scale, const kk_tensor* shift,
                                       const kk_tensor* alpha, const kk_tensor* recip, float eps);
/* kk_instance_norm_scale_shift (or its snake form when alpha and recip are
 * given) followed by the Cast(float) and DynamicQuantizeLinear that alone
 * read its result (ref_runtime.py:106-116, :500-508): y (uint8, x's shape),
 * y_scale (one fp32) and y_zero_point (one uint8) exactly as
 * kk_dynamic_quantize_linear gives them; the float result is recomputed
 * instead of stored.  leaky and alpha/recip exclude each other. */
int kk_instance_norm_quant(const kk_tensor* y, const kk_tensor* y_scale,
                           const kk_tensor* y_zero_point, const kk_tensor* x,
                           const kk_tensor* scale, const kk_tensor* shift,
                           const kk_tensor* alpha, const kk_tensor* recip, float eps,
                           int leaky, float leaky_alpha);
/* kk_instance_norm_quant with x's leaf sums from the convolution that
 * produced it (kk_conv_integer_scaled_qbias_packed_leaves; KK_E_ARG if they
 * were formed from another tensor): rows long enough for the block-wise
 * statistics take their means from the leaves instead of a pass over x
 * (the same bits: the same sums in the same order). */
int kk_instance_norm_quant_leaves(const kk_tensor* y, const kk_tensor* y_scale,
                                  const kk_tensor* y_zero_point, const kk_tensor* x,
                                  const kk_tensor* scale, const kk_tensor* shift,
                                  const kk_tensor* alpha, const kk_tensor* recip, float eps,
                                  int leaky, float leaky_alpha, const kk_tensor* leaves);
/* AdaIN with the style Linear fused: h = style . W + b with W [S, 2C]
 * (any strides), then kk_instance_norm_affine on x [N,C,T].  bias may be
 * NULL.  W may be f32, f16 or int8/uint8 with w_scale/w_zp (per tensor or
 * per column, as kk_gemm). */
int kk_adain(const kk_tensor* out, const kk_tensor* x, const kk_tensor* style,
             const kk_tensor* w, const kk_tensor* w_scale,
             const kk_tensor* w_zp, const kk_tensor* bias, float eps);
/* LayerNormalization / SkipLayerNormalization: op_layernorm
 * (ref_runtime.py:276-285) over axes [axis, rank), after s = x + skip
 * (+ skip_bias) when skip is given (:604-609).  scale/bias broadcast over
 * the normalised axes; bias may be NULL. */
int kk_layernorm(const kk_tensor* out, const kk_tensor* x,
                 const kk_tensor* skip, const kk_tensor* skip_bias,
                 const kk_tensor* scale, const kk_tensor* bias, int axis,
                 float eps);
/* Softmax along `axis`: op_softmax (ref_runtime.py:269-273). */
int kk_softmax(const kk_tensor* out, const kk_tensor* x, int axis);

/* ----------------------------------------------------------- contractions
 * Batched matmul out = alpha * a @ deq(w) with numpy batch broadcasting
 * (MatMul ref_runtime.py:614-615, FusedMatMul :616-622 with transA/transB
 * expressed as swapped strides).  deq(w) = (w - w_zp) * w_scale in fp32
 * for int8/uint8 w (DequantizeLinear :631-636, op_lstm.deq :154-158);
 * scale/zp are per tensor (one element) or per column (N elements).  f32
 * and f16 w take no scale.  Accumulation is fp32. */
int kk_gemm(const kk_tensor* out, const kk_tensor* a, const kk_tensor* w,
            const kk_tensor* w_scale, const kk_tensor* w_zp, float alpha);
/* Packed weights for kk_gemm: the weight side of MatMul on a DequantizeLinear
 * output or an fp16 weight (ref_runtime.py:614-615, 631-636), which the
 * reference dequantizes on every call.  A graph whose weights do not change
 * packs them at load: w [K, N] (N contiguous) fp16, or int8/uint8 less its
 * per-tensor or per-column zero point of the same type, as the bf16
 * matrix-core operands.  kk_gemm_packed_bytes gives the pack's size;
 * kk_gemm_pack writes it into `packed` (uint8, contiguous, 256-byte
 * aligned, that many bytes).  kk_gemm_packed is kk_gemm on a pack, with the
 * same results: w (the tensor the pack was made from, with the same zero
 * point) gives the shapes, and the call fails (KK_E_ARG) unless the last
 * kk_gemm_pack into `packed` read this very w and zero point.  Calls the
 * bf16 matrix cores do not take run kk_gemm's other kernels on w itself. */
int kk_gemm_packed_bytes(int64_t k, int64_t n, int w_dtype, int64_t* bytes);
int kk_gemm_pack(const kk_tensor* packed, const kk_tensor* w, const kk_tensor* w_zp);
int kk_gemm_packed(const kk_tensor* out, const kk_tensor* a, const kk_tensor* w,
                   const kk_tensor* packed, const kk_tensor* w_scale,
                   const kk_tensor* w_zp, float alpha);
/* Conv1d: op_conv1d forward (ref_runtime.py:58-82, 101-103).  x [N,Cin,L],
 * w [Cout, Cin/group, K] (f32/f16, or int8/uint8 dequantized with a
 * per-tensor or per-output-channel scale/zp), bias [Cout] or NULL. */
int kk_conv1d(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
              const kk_tensor* w_scale, const kk_tensor* w_zp,
              const kk_tensor* bias, int stride, int dilation, int pad0,
              int pad1, int group);
/* ConvTranspose1d: op_conv1d transposed (ref_runtime.py:83-99).
 * w [Cin, Cout/group, K]. */
int kk_conv_transpose1d(const kk_tensor* out, const kk_tensor* x,
                        const kk_tensor* w, const kk_tensor* w_scale,
                        const kk_tensor* w_zp, const kk_tensor* bias,
                        int stride, int dilation, int pad0, int pad1,
                        int group, int output_padding);
/* Constant Conv / ConvTranspose weights laid out once for the fp16 matrix
 * cores: the same convolutions as kk_conv1d / kk_conv_transpose1d (the
 * Conv :637-640 and ConvTranspose :646-651 branches over op_conv1d,
 * ref_runtime.py:58-103), whose weights the reference dequantizes on every
 * call.  A graph whose weights do not change between calls packs them at
 * load (fp16, or int8/uint8 less its per-tensor or per-channel int8/uint8
 * zero point; group 1).  kk_conv_packed_bytes gives the size of the pack
 * (transposed: ConvTranspose1d with this stride; else Conv1d, any stride);
 * kk_conv_pack writes it into `packed` (uint8, contiguous, 256-byte aligned,
 * that many bytes). */
int kk_conv_packed_bytes(int transposed, int64_t cin, int64_t cout, int64_t k,
                         int stride, int64_t* bytes);
int kk_conv_pack(const kk_tensor* packed, const kk_tensor* w,
                 const kk_tensor* w_zp, int transposed, int stride);
/* kk_conv1d (group 1) and kk_conv_transpose1d (group 1, dilation 1) on
 * weights packed by kk_conv_pack; w (the tensor the pack was made from,
 * with the same zero point) gives the shapes, and the call fails (KK_E_ARG)
 * unless the last kk_conv_pack into `packed` read this very w for this
 * operation and stride.  Shapes the matrix cores do not take run the fp32
 * kernels on w itself. */
int kk_conv1d_packed(const kk_tensor* out, const kk_tensor* x,
                     const kk_tensor* w, const kk_tensor* packed,
                     const kk_tensor* w_scale, const kk_tensor* w_zp,
                     const kk_tensor* bias, int stride, int dilation,
                     int pad0, int pad1);
int kk_conv_transpose1d_packed(const kk_tensor* out, const kk_tensor* x,
                               const kk_tensor* w, const kk_tensor* packed,
                               const kk_tensor* w_scale,
                               const kk_tensor* w_zp, const kk_tensor* bias,
                               int stride, int pad0, int pad1,
                               int output_padding);

/* --------------------------------------------- quantized integer path
 * DynamicQuantizeLinear (ref_runtime.py:106-116): y = clip(rint(x / scale)
 * + zp, 0, 255) with the range widened to include 0, scale = range / 255 and
 * zp = clip(rint(-min / scale)) derived in double; y uint8 like x, scale one
 * fp32, zp one uint8 (all on the device). */
int kk_dynamic_quantize_linear(const kk_tensor* y, const kk_tensor* scale,
                               const kk_tensor* zp, const kk_tensor* x);
/* MatMulInteger (ref_runtime.py:119-127): int32 (a - a_zp) @ (b - b_zp),
 * a uint8/int8 [.., M, K], b int8/uint8 [.., K, N], a_zp per tensor, b_zp
 * per tensor or per column (either may be NULL).  Exact integer
 * arithmetic modulo 2^32, as numpy's int32 matmul. */
int kk_matmul_integer(const kk_tensor* out, const kk_tensor* a, const kk_tensor* b,
                      const kk_tensor* a_zp, const kk_tensor* b_zp);
/* The graph's quantised-linear tail fused into MatMulInteger's epilogue:
 * MatMulInteger -> Cast(float) -> Mul(scale) (-> Add(bias)), the scale
 * itself the Mul of the activation's and the weights' scales
 * (ref_runtime.py:119-127, 572-578, 446-451): out fp32 [.., M, N] =
 * float(int32 result) * (scale[n] * scale2[n]) (+ bias[n]), each Mul and
 * the Add rounded separately as the chain does; scale, scale2 and bias
 * contiguous fp32 holding 1 or N values (scale2 and bias may be NULL);
 * K >= 1. */
int kk_matmul_integer_scaled(const kk_tensor* out, const kk_tensor* a, const kk_tensor* b,
                             const kk_tensor* a_zp, const kk_tensor* b_zp,
                             const kk_tensor* scale, const kk_tensor* scale2,
                             const kk_tensor* bias);
/* A constant [K, N] B of MatMulInteger laid out once for the int8 matrix
 * cores: the reference's op_matmul_integer (ref_runtime.py:119-127) reads
 * b as it is on every call; a graph whose weights do not change between
 * calls packs them at load.  kk_matmul_integer_pack_bytes gives the size of
 * the uint8 buffer (256-byte aligned) kk_matmul_integer_pack fills from b
 * (int8 or uint8): the fragments of every 32-column, 32-k tile in the
 * matrix cores' lane order, then the int32 column sums. */
int kk_matmul_integer_pack_bytes(const kk_tensor* b, size_t* bytes);
int kk_matmul_integer_pack(const kk_tensor* packed, const kk_tensor* b);
/* kk_matmul_integer and kk_matmul_integer_scaled on a packed B: the same
 * results bit for bit, in one launch of a kernel that loads the packed
 * fragments straight into registers.  b is the tensor the pack was made
 * from (KK_E_ARG otherwise); where A or out is not contiguous, or K is not
 * a multiple of 16, the call runs the unpacked kernel on b. */
int kk_matmul_integer_packed(const kk_tensor* out, const kk_tensor* a, const kk_tensor* b,
                             const kk_tensor* packed, const kk_tensor* a_zp,
                             const kk_tensor* b_zp);
int kk_matmul_integer_scaled_packed(const kk_tensor* out, const kk_tensor* a,
                                    const kk_tensor* b, const kk_tensor* packed,
                                    const kk_tensor* a_zp, const kk_tensor* b_zp,
                                    const kk_tensor* scale, const kk_tensor* scale2,
                                    const kk_tensor* bias);
/* ConvInteger (ref_runtime.py:130-134): int32 conv of (x - x_zp) with
 * (w - w_zp); x uint8 [N, Cin, L], w uint8/int8 [Cout, Cin, K]; padding
 * reads 0 after the zero-point shift. */
int kk_conv_integer(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                    const kk_tensor* x_zp, const kk_tensor* w_zp, int stride,
                    int dilation, int pad0, int pad1, int group);
/* The graph's quantised-conv tail fused into ConvInteger's epilogue:
 * ConvInteger -> Add(bias, int32) -> Cast(float) -> Mul(scale)
 * (ref_runtime.py:130-134, :446-455, :572-578):
 *   out[n, co, l] = float(conv_int(x, w)[n, co, l] + bias[co]) * scale
 * with out fp32, bias int32 holding Cout values or NULL, scale fp32 holding
 * 1 or Cout values.  Same integer arithmetic as kk_conv_integer. */
int kk_conv_integer_scaled(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                           const kk_tensor* x_zp, const kk_tensor* w_zp, const kk_tensor* bias,
                           const kk_tensor* scale, int stride, int dilation, int pad0, int pad1,
                           int group);
/* The same with the graph's per-call bias quantisation ahead of it folded in
 * (ref_runtime.py:450-455 Mul/Div, 472-473 Floor, 572-578 Cast): scale = Mul(scale_a,
 * scale_w) and bias_int32 = Cast(Floor(Div(bias, scale))), each rounded as
 * its node rounds it, then the conv tail as above with that bias and scale;
 * scale_a and scale_w one fp32 each, bias fp32 with Cout values. */
int kk_conv_integer_scaled_qbias(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                                 const kk_tensor* x_zp, const kk_tensor* w_zp,
                                 const kk_tensor* bias, const kk_tensor* scale_a,
                                 const kk_tensor* scale_w, int stride, int dilation, int pad0,
                                 int pad1, int group);

/* The quantised conv's output read only by an Add whose other operand has
 * the output's shape (the decoder's residual sums), the Add fused into the
 * epilogue (ref_runtime.py:446-447: Add, out = x + y in fp32):
 *   out = float(conv_int + bias) * scale + resid
 * the conv tail's value rounded as before, then the Add's one rounding;
 * resid fp32, contiguous, shaped like out (it may be out itself). */
int kk_conv_integer_scaled_add(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                               const kk_tensor* x_zp, const kk_tensor* w_zp, const kk_tensor* bias,
                               const kk_tensor* scale, const kk_tensor* resid, int stride,
                               int dilation, int pad0, int pad1, int group);
/* kk_conv_integer_scaled_qbias with the same residual Add fused in. */
int kk_conv_integer_scaled_qbias_add(const kk_tensor* out, const kk_tensor* x, const kk_tensor* w,
                                     const kk_tensor* x_zp, const kk_tensor* w_zp,
                                     const kk_tensor* bias, const kk_tensor* scale_a,
                                     const kk_tensor* scale_w, const kk_tensor* resid, int stride,
                                     int dilation, int pad0, int pad1, int group);

/* ConvInteger's weight re-layout (ref_runtime.py:130-134 reads w as it is;
 * the int8 matrix cores take it offset to int8, in fragment order, with
 * per-channel sums and zero points) done once for weights that do not change
 * between calls, e.g. a graph's constants.  kk_conv_integer_packed_bytes
 * gives the size of the packed form of a [cout, cin, k] weight;
 * kk_conv_integer_pack writes it into `packed` (uint8, contiguous, 256-byte
 * aligned, exactly that many bytes) from w (uint8/int8 [Cout, Cin, K]) and
 * its zero point (NULL: 0). */
int kk_conv_integer_packed_bytes(int64_t cout, int64_t cin, int64_t k, int64_t* bytes);
int kk_conv_integer_pack(const kk_tensor* packed, const kk_tensor* w, const kk_tensor* w_zp);
/* kk_conv_integer_scaled_qbias (resid NULL) or kk_conv_integer_scaled_qbias_add
 * (resid given) on weights packed by kk_conv_integer_pack from this w and
 * w_zp: the same checks and bit-identical results, without the per-call
 * re-layout (w and w_zp give the shapes and are not read; the caller keeps
 * `packed` in step with their contents).  A `packed` buffer is refused
 * (KK_E_ARG) unless the last kk_conv_integer_pack into it read this very w
 * (address, shape, dtype) and w_zp (address, dtype).  The per-call bias
 * quantisation is formed per block with the same operations. */
int kk_conv_integer_scaled_qbias_packed(const kk_tensor* out, const kk_tensor* x,
                                        const kk_tensor* w, const kk_tensor* packed,
                                        const kk_tensor* x_zp, const kk_tensor* w_zp,
                                        const kk_tensor* bias, const kk_tensor* scale_a,
                                        const kk_tensor* scale_w, const kk_tensor* resid,
                                        int stride, int dilation, int pad0, int pad1, int group);
/* kk_conv_integer_scaled_qbias_packed that also forms, for the InstanceNorm
 * that reads its output, the output's numpy-order leaf sums (no counterpart
 * in the reference, whose InstanceNorm chain re-reads the conv output:
 * ref_runtime.py:446-459 ReduceMean): leaves fp32 contiguous [N * Cout,
 * (Lout / 8192) * 64], leaf t of a row = np.add.reduce of its elements
 * 128 t .. 128 t + 127 (8 accumulators of 16 terms in order, then their
 * balanced tree), for the rows' whole 8192-blocks.  Lout >= 8192. */
int kk_conv_integer_scaled_qbias_packed_leaves(
    const kk_tensor* out, const kk_tensor* x, const kk_tensor* w, const kk_tensor* packed,
    const kk_tensor* x_zp, const kk_tensor* w_zp, const kk_tensor* bias, const kk_tensor* scale_a,
    const kk_tensor* scale_w, const kk_tensor* resid, const kk_tensor* leaves, int stride,
    int dilation, int pad0, int pad1, int group);

/* kk_conv_integer_scaled_qbias without any allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The same checks, kernels and results; the per-call workspace
 * (the re-laid weights and per-channel constants, normally from the pool)
 * lives in a fixed 8 MiB device array that each GPU holds from kk_init to the
 * end of the process.  A convolution whose workspace exceeds it
 * (CoutP * K * CinP + 4 * CoutP * 4 bytes, CoutP = Cout rounded up to 128,
 * CinP = Cin rounded up to 64; the Kokoro graph's largest is 3.4 MiB) is
 * rejected with KK_E_UNSUPPORTED.  Every call on a GPU shares that array:
 * calls that overlap on one GPU (e.g. from other streams or threads) race. */
int kk_conv_integer_scaled_qbias_noalloc(const kk_tensor* out, const kk_tensor* x,
                                         const kk_tensor* w, const kk_tensor* x_zp,
                                         const kk_tensor* w_zp, const kk_tensor* bias,
                                         const kk_tensor* scale_a, const kk_tensor* scale_w,
                                         int stride, int dilation, int pad0, int pad1, int group);

/* ------------------------------------------------ recurrent / vocoder
 * DynamicQuantizeLSTM as op_lstm computes it without activation
 * quantisation (ref_runtime.py:137-210): W int8 [dir, input, 4H] and R int8
 * [dir, H, 4H] dequantised ((q - zp) * scale, per direction), gate order
 * i, o, f, c, the reverse direction walking time backwards.  ys [seq, dir,
 * batch, H]; yh/yc [dir, batch, H] may be NULL; b [dir, 8H], init_h/init_c
 * [dir, batch, H] and w_zp/r_zp may be NULL.  4H <= 1024. */
int kk_lstm(const kk_tensor* ys, const kk_tensor* yh, const kk_tensor* yc,
            const kk_tensor* x, const kk_tensor* w, const kk_tensor* r,
            const kk_tensor* b, const kk_tensor* init_h, const kk_tensor* init_c,
            const kk_tensor* w_scale, const kk_tensor* w_zp, const kk_tensor* r_scale,
            const kk_tensor* r_zp, int hidden_size, int bidirectional);
/* STFT (op_stft, ref_runtime.py:213-233): direct DFT of windowed frames,
 * out [batch, frames, bins, 2]. */
int kk_stft(const kk_tensor* out, const kk_tensor* signal, const kk_tensor* window,
            int64_t frame_step, int64_t frame_length, int onesided);
/* Resize of the last axis (op_resize, ref_runtime.py:236-256): mode 0
 * nearest (asymmetric, floor), 1 linear (half_pixel); out length
 * floor(L * scale). */
int kk_resize(const kk_tensor* out, const kk_tensor* x, int mode, double scale);
/* Pad (op_pad, ref_runtime.py:259-266): pads = [begin_0.., end_0..] (host
 * array of 2*rank), mode 0 constant, 1 reflect, 2 edge. */
int kk_pad(const kk_tensor* out, const kk_tensor* x, const int64_t* pads, int mode,
           float value);
/* CumSum along `axis` (ref_runtime.py:565-567), fp32/int32/int64, summed
 * sequentially as numpy does. */
int kk_cumsum(const kk_tensor* out, const kk_tensor* x, int axis);
/* ScatterND (op_scatternd, ref_runtime.py:296-304) after the copy of data
 * into out: out[offsets[i] .. + inner] = updates[i]; offsets are host
 * element offsets, distinct and checked against out. */
int kk_scatter_nd(const kk_tensor* out, const kk_tensor* updates, const int64_t* offsets,
                  int64_t nidx, int64_t inner);

/* -------------------------------------------------- audio output stage
 * The product's output stage, KokoroAudio.stream_from_gpu
 * (addons/best-tts/runtime/audio.gd:59-106).
 * Notch FIR (kernels/fir.glsl:35-47): out[i] = sum_k taps[k] *
 * x[clamp(i - center + k, 0, n - 1)] over the flattened waveform, each
 * output's taps accumulated in order in fp32; center < 0 selects
 * (taps - 1) / 2, as audio.gd passes it.  x and out contiguous fp32 of equal
 * size, 16-byte aligned; 1 <= taps <= 4096. */
int kk_fir(const kk_tensor* out, const kk_tensor* x, const kk_tensor* taps, int center);
/* 16-bit PCM (kernels/pcm16.glsl:28-46): sample i becomes
 * round(clamp(x[i] * gain, -1, 1) * 32767) as int16 (a .5 tie rounds away
 * from zero), stored as the little-endian byte stream the reference reads
 * back: out_bytes uint8 with 2 * numel(x) elements, 16-byte aligned. */
int kk_pcm16(const kk_tensor* out_bytes, const kk_tensor* x, float gain);
/* kk_fir followed by kk_pcm16 in one pass (the FIR's fp32 result never
 * reaches memory), as audio.gd:76-99 applies them in turn. */
int kk_fir_pcm16(const kk_tensor* out_bytes, const kk_tensor* x, const kk_tensor* taps,
                 int center, float gain);

/* -------------------------------------------------------------- timing
 * HIP events on the library stream, for measuring kernels where they run.
 * Slots 0..KK_MAX_EVENTS-1.  No counterpart in the reference, which has no
 * GPU timestamps (only Time.get_ticks_msec on the host). */
#define KK_MAX_EVENTS 16
int kk_event_record(int slot);
int kk_event_elapsed(int start_slot, int stop_slot, float* ms);

/* ---------------------------------------------------------- HIP graphs
 * Records the ops called between kk_graph_begin and kk_graph_end on the
 * library stream into a HIP graph that kk_graph_launch replays -- the
 * replacement for the reference's recorded Vulkan compute list
 * (addons/best-tts/runtime/gpu.gd:227-262) when a node sequence repeats.
 * While recording, kk_alloc/kk_upload/kk_download/kk_sync fail: every
 * buffer a graph touches must exist before kk_graph_begin and stay
 * allocated while the graph may be launched. */
int kk_graph_begin(void);
/* Records as kk_graph_begin does, into a graph that owns `arena_bytes` of
 * device memory: while recording, kk_alloc hands out the arena's blocks
 * (bucketed, a block freed by one op is reused by a later one), kk_upload
 * records its bytes as arguments of copy kernels (the host buffer may change
 * after the call), and a pool buffer freed by an op is held by the graph,
 * whose replays read it again.  The arena's blocks and the held buffers go
 * back with kk_graph_destroy (kk_free of an arena block is a no-op until
 * then); kk_alloc fails with KK_E_NOMEM when the arena is used up.  This
 * lets a walk of graph nodes that allocates its intermediates, the text
 * part of a run, be recorded as it runs and replayed for the next input of
 * the same length (executor.gd:306-331 walks the nodes on every run). */
int kk_graph_begin_arena(size_t arena_bytes);
/* Ends a recording without making a graph, or follows a kk_graph_end that
 * failed on an arena recording (which keeps the arena, since the caller may
 * still hold its blocks): the arena and the held buffers are released
 * (nothing recorded has run). */
int kk_graph_abort(void);
int kk_graph_end(int* graph_id);
int kk_graph_launch(int graph_id);
int kk_graph_destroy(int graph_id);
/* Nodes of a recorded graph (every kernel an op recorded is one node). */
int kk_graph_nodes(int graph_id, int64_t* nodes);

/* ---------------------------------------------------------- dispatches
 * Kernels the library has launched since kk_init, outside graph recording
 * (a graph replay's kernels are not counted here) -- the counterpart of
 * the reference executor's per-run dispatch count
 * (addons/best-tts/runtime/executor.gd:65, 303, 356). */
int kk_dispatch_count(uint64_t* dispatches);

#ifdef __cplusplus
}
#endif
#endif /* KK_H */
