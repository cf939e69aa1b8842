/*
 * hk.h - C ABI of the MI355X (gfx950) transformer-training kernel surface.
 *
 * Every entry point replaces one kernel (or one family of template instantiations) of
 * BlubridgeAI/HyperKernels. The reference kernels are templated `__global__` functions that
 * the caller launches itself with `<<<grid, block, smem>>>`; here the library owns the launch
 * geometry, so a caller passes only the problem arguments plus a stream. Template parameters
 * (element type, layout, split-K, causal) become symbol suffixes or plain arguments.
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers (HBM) unless stated otherwise; the caller owns them.
 *   - bf16 and fp16 tensors and scalars are passed as raw bit patterns (`hk_bf16`,
 *     `hk_f16` = uint16_t).
 *   - Matrices are row-major, as in the reference harnesses.
 *   - The return value is the launch status. Nothing synchronises the stream.
 *   - Preconditions that the kernels still need are validated and reported as
 *     hipErrorInvalidValue; preconditions of the reference that this build lifts are listed
 *     at each entry point.
 */
#ifndef HK_H_
#define HK_H_

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Exported symbols of libhk_amd.so (the library is built with hidden default visibility). */
#if defined(__GNUC__)
#define HK_API __attribute__((visibility("default")))
#else
#define HK_API
#endif

typedef uint16_t hk_bf16;
typedef uint16_t hk_f16; /* IEEE binary16 bit pattern (__half) */

/* ------------------------------------------------------------------------------------------
 * Library
 * ---------------------------------------------------------------------------------------- */

/* ABI version of this header; bumped on any incompatible change. */
#define HK_ABI_VERSION 1
HK_API int hk_abi_version(void);
/* Text of a status returned by any entry point (hipGetErrorString of the library's runtime). */
HK_API const char* hk_error_string(hipError_t status);

/* ------------------------------------------------------------------------------------------
 * GELU (tanh approximation), math in fp32, accurate tanh.
 * Replaces gelu_forward_sm89_kernel<T>      (kernels/gelu/gelu_forward_sm89_kernel.cu:35-37)
 *      and OwnTensor::cuda::gelu_backward_sm89_kernel<T>
 *                                           (kernels/gelu/gelu_backward_sm89_kernel.cu:44-47).
 * Any numel and any alignment (the reference needs float4 / bf16x2 alignment).
 * ---------------------------------------------------------------------------------------- */
HK_API hipError_t hk_gelu_forward_f32(const float* in, float* out, int64_t numel, hipStream_t stream);
HK_API hipError_t hk_gelu_forward_bf16(const hk_bf16* in, hk_bf16* out, int64_t numel,
                                hipStream_t stream);
HK_API hipError_t hk_gelu_backward_f32(const float* grad, const float* in, float* grad_in,
                                int64_t numel, hipStream_t stream);
HK_API hipError_t hk_gelu_backward_bf16(const hk_bf16* grad, const hk_bf16* in, hk_bf16* grad_in,
                                 int64_t numel, hipStream_t stream);
/* fp16 forms: the reference's <__half> instantiations (gelu_forward_sm89_kernel.cu:79;
 * gelu_backward_sm89_kernel.cu:89). fp32 math, results rounded to nearest even. */
HK_API hipError_t hk_gelu_forward_f16(const hk_f16* in, hk_f16* out, int64_t numel,
                               hipStream_t stream);
HK_API hipError_t hk_gelu_backward_f16(const hk_f16* grad, const hk_f16* in, hk_f16* grad_in,
                                int64_t numel, hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * LayerNorm, fp32.
 * Forward replaces layer_norm_forward_sm89_kernel<float,float>
 *   (kernels/layernorm/layer_norm_forward_sm89_kernel.cu:27-32). The reference takes the row
 *   count from gridDim.x; here it is the `rows` argument. gamma, beta, mean_out and rstd_out
 *   may be NULL, as in the reference. Lifts the reference's blockDim == 512 requirement.
 * Backward-input replaces OwnTensor::cuda::ln_backward_input_sm89_kernel<float>
 *   (kernels/layernorm/ln_backward_input_sm89_kernel.cu:33-38); gamma may be NULL.
 * Backward-gamma/beta replaces ln_backward_gamma_beta_sm89_kernel<float>
 *   (kernels/layernorm/ln_backward_gamma_beta_sm89_kernel.cu:15-21). As in the reference the
 *   result is ADDED to grad_gamma / grad_beta (the reference adds with atomics into
 *   caller-zeroed buffers); here the sum is formed in a fixed order, so it is deterministic.
 * The fused backward computes grad_x and adds into grad_gamma / grad_beta in one pass over
 *   dy and x (no counterpart in the reference, which reads dy and x twice).
 * ---------------------------------------------------------------------------------------- */
HK_API hipError_t hk_layer_norm_forward_f32(const float* x, const float* gamma, const float* beta,
                                     float* y, float* mean_out, float* rstd_out, int rows,
                                     int cols, float eps, hipStream_t stream);
HK_API hipError_t hk_ln_backward_input_f32(const float* grad_y, const float* x, const float* mean,
                                    const float* rstd, const float* gamma, float* grad_x,
                                    int rows, int cols, hipStream_t stream);
HK_API hipError_t hk_ln_backward_gamma_beta_f32(const float* grad_y, const float* x, const float* mean,
                                         const float* rstd, float* grad_gamma, float* grad_beta,
                                         int rows, int cols, hipStream_t stream);
HK_API hipError_t hk_layer_norm_backward_f32(const float* grad_y, const float* x, const float* mean,
                                      const float* rstd, const float* gamma, float* grad_x,
                                      float* grad_gamma, float* grad_beta, int rows, int cols,
                                      hipStream_t stream);

/* The same four entry points for bf16 and fp16 tensors, replacing the reference's
 * <__nv_bfloat16, float> and <__half, float> instantiations
 *   (layer_norm_forward_sm89_kernel.cu:207-210; ln_backward_input_sm89_kernel.cu:109-113;
 *   ln_backward_gamma_beta_sm89_kernel.cu:53-56).
 * x, gamma, beta, y, grad_y and grad_x are 16-bit; mean, rstd, grad_gamma and grad_beta are
 * fp32, as in the reference. All arithmetic is fp32; y and grad_x are rounded to nearest even. */
HK_API hipError_t hk_layer_norm_forward_bf16(const hk_bf16* x, const hk_bf16* gamma, const hk_bf16* beta,
                                      hk_bf16* y, float* mean_out, float* rstd_out, int rows,
                                      int cols, float eps, hipStream_t stream);
HK_API hipError_t hk_ln_backward_input_bf16(const hk_bf16* grad_y, const hk_bf16* x, const float* mean,
                                     const float* rstd, const hk_bf16* gamma, hk_bf16* grad_x,
                                     int rows, int cols, hipStream_t stream);
HK_API hipError_t hk_ln_backward_gamma_beta_bf16(const hk_bf16* grad_y, const hk_bf16* x,
                                          const float* mean, const float* rstd,
                                          float* grad_gamma, float* grad_beta, int rows,
                                          int cols, hipStream_t stream);
HK_API hipError_t hk_layer_norm_backward_bf16(const hk_bf16* grad_y, const hk_bf16* x, const float* mean,
                                       const float* rstd, const hk_bf16* gamma, hk_bf16* grad_x,
                                       float* grad_gamma, float* grad_beta, int rows, int cols,
                                       hipStream_t stream);
HK_API hipError_t hk_layer_norm_forward_f16(const hk_f16* x, const hk_f16* gamma, const hk_f16* beta,
                                      hk_f16* y, float* mean_out, float* rstd_out, int rows,
                                      int cols, float eps, hipStream_t stream);
HK_API hipError_t hk_ln_backward_input_f16(const hk_f16* grad_y, const hk_f16* x, const float* mean,
                                     const float* rstd, const hk_f16* gamma, hk_f16* grad_x,
                                     int rows, int cols, hipStream_t stream);
HK_API hipError_t hk_ln_backward_gamma_beta_f16(const hk_f16* grad_y, const hk_f16* x,
                                          const float* mean, const float* rstd,
                                          float* grad_gamma, float* grad_beta, int rows,
                                          int cols, hipStream_t stream);
HK_API hipError_t hk_layer_norm_backward_f16(const hk_f16* grad_y, const hk_f16* x, const float* mean,
                                       const float* rstd, const hk_f16* gamma, hk_f16* grad_x,
                                       float* grad_gamma, float* grad_beta, int rows, int cols,
                                       hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * Sparse cross-entropy over fp32 logits [batch_size, vocab_size] with int32 targets.
 * Forward replaces sparse_ce_forward_kernel_vec_save_stats<float,int32_t>
 *   (kernels/loss/sparse_ce_forward_kernel_vec_save_stats.cu:14-23): per row
 *   loss = log(sum) + max - logits[target], and saves max and sum = sum_j exp(x_j - max).
 * Backward replaces sparseCENormalize_from_stats<float,int32_t>
 *   (kernels/loss/sparseCENormalize_from_stats.cu:7-17):
 *   grad = (exp(x - max) / sum - [j == target]) * (*grad_output * host_scale).
 * Both accept any vocab_size (the reference needs vocab_size % 4 == 0). A target outside
 * [0, vocab_size) gives a NaN loss and no one-hot term (the reference reads out of bounds).
 * ---------------------------------------------------------------------------------------- */
HK_API hipError_t hk_sparse_ce_forward_f32_i32(const float* logits, const int32_t* targets,
                                        float* losses, float* saved_max, float* saved_sum,
                                        int64_t batch_size, int64_t vocab_size,
                                        hipStream_t stream);
HK_API hipError_t hk_sparse_ce_backward_f32_i32(const float* logits, const int32_t* targets,
                                         float* grad, const float* saved_max,
                                         const float* saved_sum, int64_t batch_size,
                                         int64_t vocab_size, const float* grad_output,
                                         float host_scale, hipStream_t stream);

/* The same two kernels with int64 and uint16 targets, replacing the reference's
 * <float,int64_t> and <float,uint16_t> instantiations
 *   (sparse_ce_forward_kernel_vec_save_stats.cu:110-113; sparseCENormalize_from_stats.cu:55-60).
 * Arguments and results are as for the int32 forms; the target is widened to int64 before the
 * range check, so a negative int64 target also gives a NaN loss. */
HK_API hipError_t hk_sparse_ce_forward_f32_i64(const float* logits, const int64_t* targets,
                                        float* losses, float* saved_max, float* saved_sum,
                                        int64_t batch_size, int64_t vocab_size,
                                        hipStream_t stream);
HK_API hipError_t hk_sparse_ce_backward_f32_i64(const float* logits, const int64_t* targets,
                                         float* grad, const float* saved_max,
                                         const float* saved_sum, int64_t batch_size,
                                         int64_t vocab_size, const float* grad_output,
                                         float host_scale, hipStream_t stream);
HK_API hipError_t hk_sparse_ce_forward_f32_u16(const float* logits, const uint16_t* targets,
                                        float* losses, float* saved_max, float* saved_sum,
                                        int64_t batch_size, int64_t vocab_size,
                                        hipStream_t stream);
HK_API hipError_t hk_sparse_ce_backward_f32_u16(const float* logits, const uint16_t* targets,
                                         float* grad, const float* saved_max,
                                         const float* saved_sum, int64_t batch_size,
                                         int64_t vocab_size, const float* grad_output,
                                         float host_scale, hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * Multi-tensor Adam/AdamW, fp32 (decoupled weight decay inside lr * (...)):
 *   m = fmaf(b1, m, (1-b1) g); v = fmaf(b2, v, (1-b2) g g);
 *   p = p - lr * ((m / bc1) / (sqrtf(v / bc2) + eps) + wd * p)
 * hk_multi_tensor_adam keeps the reference's by-value metadata ABI
 *   (kernels/optimizer/multi_tensor_adam_sm89_kernel.cu:8-27: at most 48 tensors and 320
 *   chunks of 32768 elements per launch; num_blocks = chunks used).
 * The plan API has no counterpart in the reference: it stores the tensor/chunk table of any
 * number of tensors in device memory once, and each step is then one launch.
 * ---------------------------------------------------------------------------------------- */
#define HK_ADAM_CHUNK_SIZE 32768
#define HK_ADAM_MAX_BLOCKS 320
#define HK_ADAM_MAX_TENSORS 48
typedef struct hk_adam_launch_metadata {
  float* params[HK_ADAM_MAX_TENSORS];
  float* grads[HK_ADAM_MAX_TENSORS];
  float* ms[HK_ADAM_MAX_TENSORS];
  float* vs[HK_ADAM_MAX_TENSORS];
  int64_t sizes[HK_ADAM_MAX_TENSORS];
  unsigned char block_to_tensor[HK_ADAM_MAX_BLOCKS];
  int block_to_chunk[HK_ADAM_MAX_BLOCKS];
} hk_adam_launch_metadata;

HK_API hipError_t hk_multi_tensor_adam(const hk_adam_launch_metadata* meta, int num_blocks, float lr,
                                float beta1, float beta2, float eps, float weight_decay,
                                float bias_correction1, float bias_correction2,
                                hipStream_t stream);

typedef struct hk_adam_plan hk_adam_plan;
/* params/grads/ms/vs/sizes are HOST arrays of num_tensors device pointers / sizes. */
HK_API hipError_t hk_adam_plan_create(int num_tensors, float* const* params, float* const* grads,
                               float* const* ms, float* const* vs, const int64_t* sizes,
                               hk_adam_plan** plan_out);
HK_API hipError_t hk_adam_plan_step(const hk_adam_plan* plan, float lr, float beta1, float beta2,
                             float eps, float weight_decay, float bias_correction1,
                             float bias_correction2, hipStream_t stream);
HK_API hipError_t hk_adam_plan_destroy(hk_adam_plan* plan);
/* Chunks and launches that one step of the plan uses (for reporting). */
HK_API int64_t hk_adam_plan_num_chunks(const hk_adam_plan* plan);

/* ------------------------------------------------------------------------------------------
 * Unified sum reduction, fp32 in / fp32 out.
 * Replaces detail::ReductionLayout + build_reduce_config + launch_reduce_kernel
 *   (kernels/reduction/unified_reduce_standalone.cu:46-56, 151-221, 702-804).
 * Paths (same enum order as ReductionLayout::Path):
 *   HK_REDUCE_INNER   out[o] = sum_k src[o * input_outer_stride + k],  k < reduced_count
 *                     (input_outer_stride 0 means reduced_count, i.e. contiguous rows)
 *   HK_REDUCE_OUTER   out[o] = sum_k src[(o / inner_count) * input_outer_stride
 *                                        + (o % inner_count) + k * input_row_stride]
 *                     (a leading-axis reduction has num_outputs == inner_count; a middle-axis
 *                     one has input_outer_stride = the slab stride, as in :393-401)
 *   HK_REDUCE_GENERIC out[o] = sum_k src[in_offset(k) + out_offset(o)] with the strided
 *                     offsets given by hk_reduce_generic_f32 (the reference's
 *                     OffsetCalculator pair, :224-249).
 * Unlike the reference launcher, no device memory is allocated or freed per call: the
 * multi-workgroup partials use a workspace the library keeps per device.
 * ---------------------------------------------------------------------------------------- */
#define HK_REDUCE_INNER 0
#define HK_REDUCE_OUTER 1
#define HK_REDUCE_GENERIC 2
typedef struct hk_reduction_layout {
  int32_t path;
  int64_t num_outputs;
  int64_t reduced_count;
  int64_t input_outer_stride;
  int64_t inner_count;
  int64_t input_row_stride;
} hk_reduction_layout;

HK_API hipError_t hk_unified_reduce_sum_f32(const hk_reduction_layout* layout, const float* src,
                                     float* dst, hipStream_t stream);
/* hk_unified_reduce_sum_f32 without any allocation. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc). Same arguments, plan and results (bit for bit) as
 * hk_unified_reduce_sum_f32; the split partials live in a fixed array of
 * HK_REDUCE_NOALLOC_SCRATCH_BYTES that each device holds for the life of the process, instead
 * of the stream's grow-only workspace. The size covers every plan on a 256-CU device (the
 * largest, an outer-axis split, needs 2,095,104 bytes); a plan whose partials need more (split
 * count x num_outputs x 4 bytes, possible on a device with more CUs) returns
 * hipErrorInvalidValue before anything is launched. Calls that overlap on one device share the
 * array: they must be ordered (one stream, or events between streams). */
#define HK_REDUCE_NOALLOC_SCRATCH_BYTES (2u << 20)
HK_API hipError_t hk_unified_reduce_sum_f32_noalloc(const hk_reduction_layout* layout,
                                                    const float* src, float* dst,
                                                    hipStream_t stream);
#define HK_REDUCE_MAX_DIMS 10
HK_API hipError_t hk_reduce_generic_f32(const float* src, float* dst, int out_ndim,
                                 const int64_t* out_sizes, const int64_t* out_strides,
                                 int red_ndim, const int64_t* red_sizes,
                                 const int64_t* red_strides, hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * BF16 batched GEMM: C = alpha * op(A) op(B) + beta * C, bf16 in/out, fp32 accumulation,
 * row-major. op(A) = A [M,K] (lda >= K) or, transposed, A stored [K,M] (lda >= M);
 * op(B) = B [K,N] (ldb >= N) or, transposed, B stored [N,K] (ldb >= K). alpha/beta are bf16
 * bit patterns, applied in fp32 with one final rounding to bf16.
 * hk_bgemm replaces bgemm_NN_kernel<transA, transB> (NN/NT/TN/TT;
 *   blas/bf16/bgemm_nn_128x128_sm89_kernel.cu:23-32, trans = mycublasOperation_t: 0 = N,
 *   1 = T, 2 = C treated as T) and bgemm_NN_128x128_64x3_kernel (…_64x3_sm89_kernel.cu:23).
 * hk_bgemm_core replaces bgemm_backward_template_kernel<Cfg, Aligned, SplitK, Layout>
 *   (blas/bf16/bgemm_core_template.cu:61-70); layout is HK_LAYOUT_{NT,TN,NN} (the reference's
 *   BgemmLayout order, :59). splitK > 1 sums fp32 partials in split order (the reference adds
 *   bf16 atomics), so the result does not depend on splitK beyond fp32 rounding.
 * hk_bgemm_nt_backward (dA = dY * B^T) replaces bgemm_nt_backward_kernel
 *   (blas/bf16/bgemm_backward_nt_sm89_kernel.cu:23-32); hk_bgemm_tn_backward (dB = A^T * dY)
 *   replaces bgemm_tn_backward_kernel (blas/bf16/bgemm_backward_tn_sm89_kernel.cu:25-34).
 * hk_bgemm and the two backward entry points have no split argument (as in the reference); when
 *   the output has too few 256 x 256 tiles to fill the device the library may split K itself,
 *   where its cost model expects that to pay (same fp32 partials and split-order sum as
 *   hk_bgemm_core).
 * hk_bgemm_split_count (no counterpart in the reference: a host-only planning query for callers
 *   and tests that check which plan runs) returns the number of k splits a product of this
 *   shape runs with (contiguous operands, 16-byte aligned): splitK = 0 for hk_bgemm and the
 *   backward entry points (the library's choice), the hk_bgemm_core argument otherwise. 1 for
 *   the GEMV and fallback kernels, 0 for an empty product, -1 for an invalid argument.
 * Any M, N, K; the MFMA path needs the contiguous extents, leading dimensions and strides to
 * be multiples of 8 and 16-byte aligned pointers (the reference's own precondition,
 * bgemm_test.cu:252-256); other shapes run on a slower fp32-accumulating kernel.
 * ---------------------------------------------------------------------------------------- */
#define HK_LAYOUT_NT 0
#define HK_LAYOUT_TN 1
#define HK_LAYOUT_NN 2
HK_API hipError_t hk_bgemm(int transA, int transB, int M, int N, int K, hk_bf16 alpha,
                           const hk_bf16* A, int lda, long long strideA, const hk_bf16* B,
                           int ldb, long long strideB, hk_bf16 beta, hk_bf16* C, int ldc,
                           long long strideC, int batchCount, hipStream_t stream);
HK_API hipError_t hk_bgemm_core(int layout, int splitK, int M, int N, int K, hk_bf16 alpha,
                                const hk_bf16* A, int lda, long long strideA, const hk_bf16* B,
                                int ldb, long long strideB, hk_bf16 beta, hk_bf16* C, int ldc,
                                long long strideC, int batchCount, hipStream_t stream);
HK_API hipError_t hk_bgemm_nt_backward(int M, int N, int K, hk_bf16 alpha, const hk_bf16* A,
                                       int lda, long long strideA, const hk_bf16* B, int ldb,
                                       long long strideB, hk_bf16 beta, hk_bf16* C, int ldc,
                                       long long strideC, int batchCount, hipStream_t stream);
HK_API hipError_t hk_bgemm_tn_backward(int M, int N, int K, hk_bf16 alpha, const hk_bf16* A,
                                       int lda, long long strideA, const hk_bf16* B, int ldb,
                                       long long strideB, hk_bf16 beta, hk_bf16* C, int ldc,
                                       long long strideC, int batchCount, hipStream_t stream);
HK_API int hk_bgemm_split_count(int transA, int transB, int M, int N, int K, int batchCount,
                                int splitK);
/* hk_bgemm_tile_rows (no counterpart in the reference: a host-only planning query, like
 * hk_bgemm_split_count) returns the rows per output tile the MFMA path runs a product of this
 * shape with: 256, or 192 when 256-row tiles would leave most CUs idle and A is k-major
 * (transA == 0); 0 for the GEMV and fallback kernels or an empty product, -1 for an invalid
 * argument. hk_bgemm_tile_cols (likewise a host-only query) returns the columns per output
 * tile: 160 when both operands are k-major (transA == 0, transB != 0), the product runs in one
 * k split, M, N and K are multiples of 256, 160 and 64, and 256 x 256 tiles would leave CUs
 * idle while 256 x 160 tiles fit one round (the 8192 x 1280 x 5120 dA product); otherwise 256
 * (the last tile columns may run 128 wide); 0 / -1 as hk_bgemm_tile_rows. */
HK_API int hk_bgemm_tile_rows(int transA, int transB, int M, int N, int K, int batchCount,
                              int splitK);
HK_API int hk_bgemm_tile_cols(int transA, int transB, int M, int N, int K, int batchCount,
                              int splitK);

/* ------------------------------------------------------------------------------------------
 * Batched BF16 GEMV, the M == 1 / N == 1 GEMMs, fp32 accumulation, one bf16 rounding.
 * Replace the four kernels of blas/bf16/bgemv_sm89_kernel.cu, same arguments in the same order
 * (the reference's Beta0 template instantiations are beta == 0 here, where C is not read):
 *   hk_bgemv_nn_row  bgemv_nn_row_vec8_kernel<Beta0> (:11-57):  C[n] = a sum_k A[k] B[k*ldb+n]
 *   hk_bgemv_nt_row  bgemv_nt_row_kernel<Beta0>      (:60-107): C[n] = a sum_k A[k] B[n*ldb+k]
 *   hk_bgemv_tn_row  bgemv_tn_row_vec8_kernel<Beta0> (:110-156): C[n] = a sum_k A[k*lda] B[k*ldb+n]
 *   hk_bgemv_nn_col  bgemv_nn_col_kernel<Beta0>      (:159-208): C[m] = a sum_k A[m*lda+k] B[k]
 *   (+ beta C[.] when beta != 0), for each of batchCount batches with element strides sA, sB,
 *   sC. Any N, M, K, strides and alignment (the reference's vec8 row kernels need N a multiple
 *   of 8 and N >= 2048, bgemm_test.cu:405-408). hk_bgemm routes its M == 1 and N == 1 products
 *   here as well.
 * ---------------------------------------------------------------------------------------- */
HK_API hipError_t hk_bgemv_nn_row(int N, int K, hk_bf16 alpha, const hk_bf16* A, const hk_bf16* B,
                                  int ldb, hk_bf16 beta, hk_bf16* C, int batchCount, long long sA,
                                  long long sB, long long sC, hipStream_t stream);
HK_API hipError_t hk_bgemv_nt_row(int N, int K, hk_bf16 alpha, const hk_bf16* A, const hk_bf16* B,
                                  int ldb, hk_bf16 beta, hk_bf16* C, int batchCount, long long sA,
                                  long long sB, long long sC, hipStream_t stream);
HK_API hipError_t hk_bgemv_tn_row(int N, int K, hk_bf16 alpha, const hk_bf16* A, int lda,
                                  const hk_bf16* B, int ldb, hk_bf16 beta, hk_bf16* C,
                                  int batchCount, long long sA, long long sB, long long sC,
                                  hipStream_t stream);
HK_API hipError_t hk_bgemv_nn_col(int M, int K, hk_bf16 alpha, const hk_bf16* A, int lda,
                                  const hk_bf16* B, hk_bf16 beta, hk_bf16* C, int batchCount,
                                  long long sA, long long sB, long long sC, hipStream_t stream);

/* BF16 GEMM with a bias, one semantics for both entry points:
 *   C = alpha * op(A) op(B) + beta * bias, C written and not read, the bias element of output
 *   (row, col) chosen by bias_numel: N -> bias[col], else M -> bias[row], else 1 -> bias[0],
 *   else M*N -> bias[row * N + col] (one M x N bias for every batch); any other bias_numel is
 *   rejected.
 * hk_bgemm_addmm replaces bgemm_addmm_kernel<BM, BN, BK, STAGES, THREADS, Aligned>
 *   (blas/bf16/bgemm_addmm_sm89_kernel.cu:15-24; epilogue :214-300), NN only, and keeps its
 *   argument order. bias == NULL gives C = alpha * A B (the kernel adds beta * 0 then); the
 *   reference's kernel accepts bias_numel 1, N and M*N, and its test computes
 *   alpha * A B + beta * bias (test_bgemm_addmm_sm89.cu:50-53, 91-94), which is what this
 *   entry point computes.
 * hk_bgemm_core_bias is hk_bgemm_core with the split-K bias initialisation of
 *   bgemm_scale_template_kernel (blas/bf16/bgemm_core_template.cu:270-289: C <- beta * bias,
 *   bias_numel N, M, 1 or M*N, before the splits accumulate): bias == NULL gives
 *   hk_bgemm_core's C = alpha * op(A) op(B) + beta * C. */
HK_API hipError_t hk_bgemm_addmm(int M, int N, int K, hk_bf16 alpha, const hk_bf16* A, int lda,
                                 long long strideA, const hk_bf16* B, int ldb, long long strideB,
                                 hk_bf16 beta, const hk_bf16* bias, int64_t bias_numel,
                                 hk_bf16* C, int ldc, long long strideC, int batchCount,
                                 hipStream_t stream);
HK_API hipError_t hk_bgemm_core_bias(int layout, int splitK, int M, int N, int K, hk_bf16 alpha,
                                     const hk_bf16* A, int lda, long long strideA,
                                     const hk_bf16* B, int ldb, long long strideB, hk_bf16 beta,
                                     const hk_bf16* bias, int64_t bias_numel, hk_bf16* C, int ldc,
                                     long long strideC, int batchCount, hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * FP32 batched GEMM with fp32-class products (the reference uses single-pass TF32; gfx950 has no
 * TF32 MFMA): a bf16x3 split on the bf16 MFMA (x = hi + lo, a b = ah bh + ah bl + al bh, relative
 * error ~1e-5) when every dimension is a multiple of 8, exact fp32 MFMA products otherwise,
 * row-major, layout HK_LAYOUT_{NT,TN,NN} as SgemmLayout (blas/fp32/sgemm_sm89_core_template.cu:9).
 * hk_sgemm replaces sgemm_sm89_kernel<Cfg, Aligned, SplitK, Layout> (…core_template.cu:85-94):
 *   C = alpha * op(A) op(B) + beta * C + bias, the bias added EXACTLY ONCE whatever splitK is
 *   (the reference's split-K path adds it once per split). bias may be NULL; otherwise
 *   bias_stride selects it as in the reference (:303-315): N -> bias[col];
 *   M*N -> bias[(batch % M) * N + col]; 1 -> bias[0]; any other value is rejected.
 *   splitK >= 1 cuts the k loop into splitK ranges as the reference does (k_chunk rounded to
 *   the k-tile, :123-126; on the bf16x3 path the tripled k axis) whose products are summed in
 *   split order: as fp32 partials with a finishing pass, or, when the output tiles alone fill
 *   the device, added into C range after range (beta and the bias with the first); splitK = 0
 *   lets the library choose. Calls that overlap on one C race. The reference's split-K pre-scale
 *   kernel sgemm_sm89_scale_kernel (:329-333) is folded in: no caller pre-pass is needed.
 * hk_sgemm_addmm replaces sgemm_addmm_sm89_kernel (blas/fp32/sgemm_addmm_sm89_kernel.cu:66-76):
 *   NN, C = alpha * A B + beta * C + beta * bias, bias_numel in {1, N, M*N} as there.
 * hk_sgemm_layout replaces every tile-specialised SGEMM kernel (sgemm_nn_256x128_sm89_2_opt_k,
 *   sgemm_nn_256x64_sm89_2_k, sgemm_nn_64x64_sm89_2_k, sgemm_nn_256x128_bypass_sm89_batched_kernel,
 *   sgemm_nt_{256x128,128x128,64x128}_sm89_2_k, sgemm_tn_256x128_sm89_optimized,
 *   sgemm_tn_{128x128,256x64}_sm89_2_k, sgemm_tn_{64x64,32x32}_sm89_k): the same product
 *   C = alpha * op(A) op(B) + beta * C for the kernel's layout (splitK as for hk_sgemm; pass 1
 *   for kernels without a splitK argument, or 0 to let the library split). The tile shape is
 *   the library's choice.
 * hk_sgemm_split_count (no counterpart in the reference: a host-only planning query) returns
 *   the number of k splits hk_sgemm / hk_sgemm_layout run for this shape and splitK
 *   (contiguous operands, 16-byte aligned): 1 on the k-order fallback, 0 for an empty product,
 *   -1 for an invalid argument. hk_sgemm_addmm runs with splitK = 0.
 * Any M, N, K; the MFMA path needs the contiguous extents, leading dimensions and strides to
 * be multiples of 4 and 16-byte aligned pointers (sgemm_test.cu:240-243); other shapes run on a
 * slower k-order kernel.
 * ---------------------------------------------------------------------------------------- */
HK_API hipError_t hk_sgemm(int layout, int M, int N, int K, float alpha, const float* A, int lda,
                           long long strideA, const float* B, int ldb, long long strideB,
                           float beta, float* C, int ldc, long long strideC, const float* bias,
                           long long bias_stride, int batchCount, int splitK, hipStream_t stream);
HK_API hipError_t hk_sgemm_addmm(int M, int N, int K, float alpha, const float* A, int lda,
                                 long long strideA, const float* B, int ldb, long long strideB,
                                 float beta, const float* bias, int64_t bias_numel, float* C,
                                 int ldc, long long strideC, int batchCount, hipStream_t stream);
HK_API hipError_t hk_sgemm_layout(int layout, int M, int N, int K, float alpha, const float* A,
                                  int lda, long long strideA, const float* B, int ldb,
                                  long long strideB, float beta, float* C, int ldc,
                                  long long strideC, int batchCount, int splitK,
                                  hipStream_t stream);
HK_API int hk_sgemm_split_count(int layout, int M, int N, int K, int batchCount, int splitK);

/* ------------------------------------------------------------------------------------------
 * Attention, fp32 I/O, head_dim 64 (the reference's only instantiation), products as a bf16x3
 * split on the bf16 MFMA (fp32-class accuracy, relative error ~1e-5; gfx950 has no TF32 MFMA).
 * Tensors are [B, nh, T, head_dim] with arbitrary batch/head/row strides (elements; last-dim
 * stride 1; strides multiples of 4 and 16-byte aligned bases), LSE and D are [B, nh, T].
 * Non-finite inputs give NaN outputs.
 * The parameter blocks repeat the reference's field order and types exactly:
 *   hk_attn_fwd_params = MemEfficientFwdParams
 *     (kernels/attention/fused_attn_forward_kernel_tc_sm89.cu:8-29);
 *   hk_attn_bwd_params = MemEfficientBwdParams
 *     (kernels/attention/mem_efficient_bwd_precompute_D_sm89.cu:7-33; the OwnTensor copy,
 *     mem_efficient_bwd_unified_kernel_exp12.cu:11-38, has the same layout).
 * hk_fused_attn_forward replaces fused_attn_forward_kernel_tc_sm89<64, 64, 64, 1> (:72-74):
 *   O = softmax(scale Q K^T [+ causal mask j <= i]) V, LSE = max + ln(sum of exp).
 *   With dropout_p > 0 and a non-NULL dropout_mask (fp32 [B*nh, T, T], contiguous, indexed
 *   (bh*T + i)*T + j as the reference does, :316-323), every exp term is multiplied by its
 *   mask value and the row sum is taken afterwards: O is normalised by the post-dropout sum
 *   and LSE = max + ln(that sum), -inf for a row with nothing kept (O = 0 there) (:326-345).
 * hk_attn_bwd_precompute_D replaces mem_efficient_bwd_precompute_D_sm89<HeadDim> (:45-91):
 *   D = rowsum(dO * O); any head_dim in [1, 256] (the reference instantiates 16, 32, 48, 64,
 *   80, 96, 128, 160, 192 and 256, :93-102) and any O / dO strides (unit last-dim stride).
 * hk_attn_backward replaces OwnTensor::mem_efficient_bwd_unified_kernel_exp12<64, Causal>
 *   (mem_efficient_bwd_unified_kernel_exp12.cu:54-56): from Q, K, V, dO, LSE and D it WRITES
 *   dK and dV and ADDS into dQ (dQ accumulates atomically across key tiles, as in the
 *   reference, so the caller zeroes dQ first; kernels_test.cu:562). is_causal selects the mask.
 * ---------------------------------------------------------------------------------------- */
typedef struct hk_attn_fwd_params {
  const float* Q;
  const float* K;
  const float* V;
  float* O;
  float* LSE;
  int B;
  int nh;
  int64_t T;
  float scale;
  bool is_causal;
  float dropout_p;
  const float* dropout_mask;
  int64_t q_strideB, q_strideM, q_strideH;
  int64_t k_strideB, k_strideM, k_strideH;
  int64_t v_strideB, v_strideM, v_strideH;
  int64_t o_strideB, o_strideM, o_strideH;
  int64_t lse_strideB, lse_strideH;
} hk_attn_fwd_params;

typedef struct hk_attn_bwd_params {
  const float* Q;
  const float* K;
  const float* V;
  const float* O;
  const float* dO;
  const float* LSE;
  float* D;
  float* dQ;
  float* dK;
  float* dV;
  int B;
  int nh;
  int T;
  float scale;
  bool is_causal;
  int64_t q_strideB, q_strideM, q_strideH;
  int64_t k_strideB, k_strideM, k_strideH;
  int64_t v_strideB, v_strideM, v_strideH;
  int64_t o_strideB, o_strideM, o_strideH;
  int64_t do_strideB, do_strideM, do_strideH;
  int64_t dq_strideB, dq_strideM, dq_strideH;
  int64_t dk_strideB, dk_strideM, dk_strideH;
  int64_t dv_strideB, dv_strideM, dv_strideH;
  int64_t lse_strideB, lse_strideH;
  int64_t d_strideB, d_strideH;
} hk_attn_bwd_params;

HK_API hipError_t hk_fused_attn_forward(const hk_attn_fwd_params* params, int head_dim,
                                        hipStream_t stream);
HK_API hipError_t hk_attn_bwd_precompute_D(const hk_attn_bwd_params* params, int head_dim,
                                           hipStream_t stream);
HK_API hipError_t hk_attn_backward(const hk_attn_bwd_params* params, int head_dim,
                                   hipStream_t stream);

/* ------------------------------------------------------------------------------------------
 * Measurement
 * ---------------------------------------------------------------------------------------- */
/* HBM stream with a given read/write mix. No counterpart in the reference: a measurement aid for
 * benchmarks, which time it to find the HBM rate a memory-bound kernel's mix can reach. Reads
 * n_in (0-4) fp32 arrays in[s] of n elements and writes n_out (0-3) arrays out[s] of n elements,
 * out[s][i] = sum over inputs of in[.][i] + s. n is a multiple of 4, every array 16-byte
 * aligned; each workgroup covers `unroll` (1, 2 or 4) spans of 256 x 16 bytes per array. With
 * n_out == 0, `sink` (one float per workgroup) must be non-NULL; it is written only if an
 * element sum equals 1234.5. The pointer arrays are read on the host. */
HK_API hipError_t hk_hbm_stream(const float* const* in, int n_in, float* const* out, int n_out,
                                int64_t n, int unroll, float* sink, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HK_H_ */
