/*
 * mx.h -- C ABI of the MI355X (gfx950) FP32 conv / GEMM / fused-AdamW library.
 *
 * Every entry point is `extern "C"`, takes plain pointers and sizes, returns an
 * int status (MX_OK == 0) and is asynchronous on the `stream` argument (a
 * hipStream_t passed as void*; NULL is HIP's null stream, as in the HIP API).
 * On failure mx_last_error() returns a thread-local message.  All validation
 * happens on the host before any launch.
 *
 * Each declaration names the reference interface it replaces
 * (mistrjirka/Pytorch-vulkan, paths relative to the repository root).
 */
#ifndef MX_H
#define MX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum mx_status {
  MX_OK = 0,
  MX_ERR_INVALID = 1,     /* bad shape / argument: TORCH_CHECK failures in the reference */
  MX_ERR_UNSUPPORTED = 2, /* forced algorithm not applicable (convolution.cpp:472-473) */
  MX_ERR_OOM = 3,         /* device allocation failed */
  MX_ERR_HIP = 4,         /* HIP runtime error */
  MX_ERR_WORKSPACE = 5    /* workspace budget too small for the requested algorithm */
};

/* ------------------------------------------------------------------------ */
/* Errors, version, device                                                   */
/* ------------------------------------------------------------------------ */

/* Thread-local message of the last failing call ("" if none). */
const char* mx_last_error(void);
int mx_abi_version(void);

/* Replaces VulkanContext::instance() device creation
 * (csrc/vulkan_context.cpp:64-83) and validate_vulkan_device. */
int mx_init(int ordinal);
int mx_device_count(int* count);
int mx_get_device(int* ordinal);
int mx_set_device(int ordinal);
int mx_device_name(int ordinal, char* buf, size_t len);
int mx_device_synchronize(void);

/* ------------------------------------------------------------------------ */
/* Streams and events: replace the single VkQueue + Kompute sequences        */
/* (csrc/torch_vulkan.cpp:34-103, csrc/vulkan_context.cpp:444-510).           */
/* ------------------------------------------------------------------------ */

/* The library's default stream of the current device (non-blocking, default
 * priority); the PrivateUse1 layer's stream 0. */
int mx_default_stream(void** stream);
int mx_stream_create(void** stream);
int mx_stream_destroy(void* stream);
int mx_stream_synchronize(void* stream);
/* *done = 1 when all work on the stream has completed. */
int mx_stream_query(void* stream, int* done);
int mx_stream_wait_event(void* stream, void* event);
int mx_event_create(void** event, int enable_timing);
int mx_event_destroy(void* event);
int mx_event_record(void* event, void* stream);
int mx_event_query(void* event, int* done);
int mx_event_synchronize(void* event);
int mx_event_elapsed_ms(void* start, void* end, float* ms);

/* ------------------------------------------------------------------------ */
/* Stream-ordered caching device allocator: replaces VulkanAllocator         */
/* (csrc/vulkan_allocator.h:22-73, csrc/vulkan_allocator.cpp:19-154).         */
/* A freed block is reusable at once by later work on its allocation stream; */
/* use on other streams (mx_record_stream) defers reuse until events recorded */
/* on those streams at free time have completed.                             */
/* ------------------------------------------------------------------------ */

typedef struct mx_memory_stats {
  uint64_t allocated_bytes;  /* bytes in live blocks */
  uint64_t reserved_bytes;   /* bytes obtained from hipMalloc and not yet released */
  uint64_t cached_blocks;    /* free blocks held for reuse */
  uint64_t device_mallocs;   /* hipMalloc calls so far */
  uint64_t cache_hits;       /* allocations served from the cache */
} mx_memory_stats;

int mx_malloc(void** ptr, size_t bytes, void* stream);
int mx_free(void* ptr);
int mx_record_stream(void* ptr, void* stream);
int mx_empty_cache(void);
int mx_memory_stats_get(mx_memory_stats* out);

enum mx_copy_kind { MX_COPY_H2D = 1, MX_COPY_D2H = 2, MX_COPY_D2D = 3 };
/* Async copy on `stream`.  D2H/H2D with pageable host memory is staged and is
 * complete on return (as the reference's ensure_host_read,
 * csrc/vulkan_context.cpp:98-112). */
int mx_memcpy(void* dst, const void* src, size_t bytes, int kind, void* stream);
/* *pinned = 1 when `ptr` lies in page-locked host memory HIP knows
 * (hipHostMalloc, including torch's pinned-memory allocator), else 0.  The
 * reference has no pinned memory (csrc/ops/mm.cpp:664 rejects pin_memory);
 * this serves non_blocking copies (torch's Tensor.to(non_blocking=True)). */
int mx_host_is_pinned(const void* ptr, int* pinned);
/* Page-locked host memory (hipHostMalloc), cached by rounded size and
 * returned to the cache by mx_host_free (released by mx_empty_cache): the
 * PrivateUse1 pinned-memory allocator behind Tensor.pin_memory(). */
int mx_host_malloc(void** ptr, size_t bytes);
int mx_host_free(void* ptr);
/* H2D / D2H copy on `stream` that returns before the copy runs (no host
 * staging).  The host side must be page-locked over its whole range (else
 * MX_ERR_INVALID) and stay alive and untouched until the stream reaches the
 * copy (record an event after it). */
int mx_memcpy_async(void* dst, const void* src, size_t bytes, int kind, void* stream);

/* ------------------------------------------------------------------------ */
/* Elementwise / layout plumbing used by the operator surface                */
/* (csrc/ops/mm.cpp:480-700, csrc/ops/native_utils.h:106-151).               */
/* ------------------------------------------------------------------------ */

/* Fill `count` elements of `elem_size` (1,2,4,8) bytes with the low bytes of
 * `pattern` (fill_.Scalar / zero_, csrc/ops/loss_primitives.cpp:374-375). */
int mx_fill(void* dst, int64_t count, int elem_size, uint64_t pattern, void* stream);

/* Strided copy of up to 8 dims: dst[idx] = src[idx] with element strides and
 * element offsets, elements of `elem_size` bytes.  This is the conv2d_pack
 * view materialisation (csrc/shaders/conv2d_pack.comp:12-22,
 * csrc/ops/convolution.cpp:62-99) and the strided device copy_
 * (csrc/ops/mm.cpp:592-608). */
int mx_copy_strided(void* dst, const void* src, int ndim, const int64_t* sizes,
                    const int64_t* dst_strides, const int64_t* src_strides,
                    int64_t dst_offset, int64_t src_offset, int elem_size, void* stream);

/* out[i] = a[i] + alpha * b[i] (FP32, contiguous): aten::add.Tensor used by
 * autograd gradient accumulation.  With b == NULL: out[i] = a[i] + alpha. */
int mx_add_f32(float* out, const float* a, const float* b, float alpha, int64_t n, void* stream);
/* out[i] = a[i] * s (FP32 contiguous): mul.Scalar (csrc/ops/mm.cpp:921-930). */
int mx_scale_f32(float* out, const float* a, float s, int64_t n, void* stream);
/* out[i] = a[i] * b[i] (FP32 contiguous): mul.Tensor on equal shapes (the
 * addmm backward's beta / alpha scaling arrives as a broadcast operand). */
int mx_mul_f32(float* out, const float* a, const float* b, int64_t n, void* stream);

/* Sum over the middle axis of a contiguous [outer, reduce, inner] FP32 view:
 * out[o, i] = sum_r src[o, r, i].  Replaces sum.dim_IntList
 * (csrc/ops/reduce.cpp:24-35), e.g. the Linear bias gradient dY.sum(0). */
int mx_sum_f32(float* out, const float* src, int64_t outer, int64_t reduce, int64_t inner,
               void* stream);

/* In-place `ptrs[i][0..numels[i]) += value` over a list of FP32 tensors in one
 * launch (_foreach_add_.Scalar on the optimizer step counters). */
int mx_foreach_add_scalar_f32(float* const* ptrs, const int64_t* numels, int64_t count,
                              float value, void* stream);

/* ------------------------------------------------------------------------ */
/* Conv2D (FP32 NCHW)                                                         */
/* ------------------------------------------------------------------------ */

/* ConvParams (csrc/ops/convolution.cpp:45-52). oh/ow are outputs of
 * mx_conv2d_check. */
typedef struct mx_conv2d_desc {
  int64_t n, cin, h, w;      /* input  [n, cin, h, w] */
  int64_t cout, kh, kw;      /* weight [cout, cin/groups, kh, kw] */
  int64_t sh, sw, ph, pw, dh, dw, groups;
  int64_t oh, ow;            /* output [n, cout, oh, ow] (filled by mx_conv2d_check) */
} mx_conv2d_desc;

enum mx_conv_phase { MX_CONV_FORWARD = 0, MX_CONV_DINPUT = 1, MX_CONV_DWEIGHT = 2, MX_CONV_DBIAS = 3 };

/* Algorithms (candidate menu of csrc/ops/convolution.cpp:161-187):
 * AUTO lets the planner choose; DIRECT is one-output-per-thread; IMPLICIT_GEMM
 * is the MFMA tile path; WINOGRAD is F(2x2,3x3) for the forward, the input
 * gradient (padding <= 2) and the weight gradient of a 3x3 stride-1
 * dilation-1 layer (the gradients are an addition: the reference's Winograd is
 * forward only); AUTO takes it in every phase for such layers with padding
 * <= 2 and >= 32 channels per group on both sides where it measures faster
 * than the implicit GEMM on MI355X: forward and input gradient from 16384
 * output positions, or from 512 when the channel walk (input channels for the
 * forward, output channels for the input gradient) is at most 4x the channels
 * produced; weight gradient from 2^25 multiply-adds per filter tap (positions
 * x input channels per group x output channels); and for the reference's
 * grouped forward rule; REDUCE is the no-scratch dWeight / dBias
 * reduction; DEPTHWISE is the forward of a layer with groups == cin and any
 * channel multiplier (conv2d_depthwise.comp:15-41; candidate rule
 * csrc/ops/convolution.cpp:361, chosen by AUTO when cin >= 8 as at :462). */
enum mx_conv_algo {
  MX_CONV_ALGO_AUTO = 0,
  MX_CONV_ALGO_DIRECT = 1,
  MX_CONV_ALGO_IMPLICIT_GEMM = 2,
  MX_CONV_ALGO_WINOGRAD = 3,
  MX_CONV_ALGO_REDUCE = 4,
  MX_CONV_ALGO_DEPTHWISE = 5
};

/* Validation and output shape: convolution_params
 * (csrc/ops/convolution.cpp:101-156).  Fills desc->oh / desc->ow. */
int mx_conv2d_check(mx_conv2d_desc* desc);

/* Algorithm the planner would run for `phase` given `requested`
 * (heuristic / applicable, csrc/ops/convolution.cpp:357-482).  Returns
 * MX_ERR_UNSUPPORTED when a forced algorithm does not apply. */
int mx_conv2d_select(const mx_conv2d_desc* desc, int phase, int requested, int* algo);

/* y = conv(x, w) + bias.  bias may be NULL (zero bias, csrc/ops/convolution.cpp:660).
 * Replaces convolution_overrideable's dispatch(Forward)
 * (csrc/ops/convolution.cpp:641-665, conv2d_tiled_body.glsl,
 * conv2d_winograd_*.comp). */
int mx_conv2d_forward(const mx_conv2d_desc* desc, const float* x, const float* w,
                      const float* bias, float* y, int algo, void* stream);

/* dx = conv_transpose(dy, w): dispatch(Input) (csrc/ops/convolution.cpp:684-687,
 * conv2d_backward_input_tiled_body.glsl).  With MX_CONV_ALGO_WINOGRAD (3x3,
 * stride 1, dilation 1, padding <= 2) dx is computed as the F(2x2,3x3)
 * convolution of dy with the spatially flipped, channel-swapped filter at
 * padding 2 - p. */
int mx_conv2d_backward_input(const mx_conv2d_desc* desc, const float* dy, const float* w,
                             float* dx, int algo, void* stream);

/* dw = sum over positions dy x im2col(x); db = sum over positions of dy.
 * Either dw or db may be NULL.  dispatch(Weight) + dispatch(Bias)
 * (csrc/ops/convolution.cpp:688-695, conv2d_backward_weight_tiled_body.glsl,
 * conv2d_backward_weight_finalize.comp, conv2d_backward_bias_reduce.comp):
 * dBias rides on the dWeight GEMM's dy operand; K splits are summed in split
 * order by a finalize launch, so the result is deterministic. */
int mx_conv2d_backward_weight(const mx_conv2d_desc* desc, const float* x, const float* dy,
                              float* dw, float* db, int algo, void* stream);

/* dx, dw and db of one layer in one call: convolution_backward's
 * dispatch(Input), dispatch(Weight) and dispatch(Bias)
 * (csrc/ops/convolution.cpp:667-697).  Any of dx, dw, db may be NULL (not
 * requested).  When both gradients of a 3x3 stride-1 layer take the fused
 * Winograd paths (algo_dx and algo_dw MX_CONV_ALGO_WINOGRAD) they run as one
 * launch, workgroups of both kinds side by side, bit-identical to
 * mx_conv2d_backward_input followed by mx_conv2d_backward_weight; otherwise
 * it is those two calls. */
int mx_conv2d_backward(const mx_conv2d_desc* desc, const float* x, const float* w, const float* dy,
                       float* dx, float* dw, float* db, int algo_dx, int algo_dw, void* stream);

/* *one_launch = 1 when mx_conv2d_backward with these arguments (dx and dw
 * requested, dBias too when with_bias != 0) runs both gradients as the one
 * Winograd launch (wino_bwd_kernel), 0 when it makes the two separate calls.
 * No data is read.  No counterpart in the reference, whose backward
 * dispatches gradient by gradient (csrc/ops/convolution.cpp:684-695): it lets
 * a caller label per-kernel timing and count launches by what runs. */
int mx_conv2d_backward_one_launch(const mx_conv2d_desc* desc, int algo_dx, int algo_dw, int with_bias,
                                  int* one_launch);

/* Allocation-free dWeight / dBias.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory while they run (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, algorithms and results as mx_conv2d_backward_weight, but
 * every scratch buffer (split-K partials, Winograd range partials, the partial
 * gradient of a batch run in chunks) lives in a library-owned device array of
 * MX_NOALLOC_SCRATCH_BYTES per GPU instead of the allocator: plans are sized
 * to fit it (and TORCH_VULKAN_CONV_WORKSPACE_MB), and a call whose smallest
 * plan still needs more fails with MX_ERR_WORKSPACE before any launch.  No
 * hipMalloc / hipFree / allocator call is made.  Every call on a GPU shares
 * that GPU's array and overwrites what it reads, so nothing needs clearing;
 * calls that overlap in time on one GPU (other streams, other threads) race
 * and must be serialised by the caller. */
#define MX_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)
int mx_conv2d_backward_weight_noalloc(const mx_conv2d_desc* desc, const float* x, const float* dy, float* dw,
                                      float* db, int algo, void* stream);

/* db only (conv2d_backward_bias_reduce.comp:10-24). */
int mx_conv2d_backward_bias(const mx_conv2d_desc* desc, const float* dy, float* db, void* stream);

/* Split-K plan of the dWeight reduction (weight_split_plan,
 * csrc/ops/convolution.cpp:204-238): number of K splits and workspace bytes
 * the implicit-GEMM dWeight path uses for this descriptor. */
int mx_conv2d_dweight_plan(const mx_conv2d_desc* desc, int64_t* splits, int64_t* span,
                           int64_t* workspace_bytes);

/* Plan of one conv call with these arguments (no data is read; operands are
 * taken to be contiguous and 256-byte aligned, as tensors from the device
 * allocator are).  The reference's planner exposes the same facts through
 * its dispatch counters and autotune plan cache (selected tile, split count,
 * split span, workspace bytes: csrc/ops/convolution.cpp:204-247, :523-639;
 * tests/test_conv_dispatch.py:255-297). */
typedef struct mx_conv2d_plan_info {
  int algo;                /* algorithm that runs (never AUTO) */
  int tile;                /* implicit-GEMM tile (index of the tile menu), -1 for other algorithms */
  int64_t splits;          /* K splits of the implicit GEMM (1: none) */
  int64_t span;            /* K per split */
  int64_t workspace_bytes; /* scratch counted against the workspace budget */
  char variant[256];       /* kernel instantiations launched, space separated */
} mx_conv2d_plan_info;

/* `with_bias` != 0 plans a dWeight call that also writes dBias.
 * Workspace budget: TORCH_VULKAN_CONV_WORKSPACE_MB (integer MiB in [0, 4096],
 * default 64; csrc/ops/convolution.cpp:239-247) caps the split-K partials,
 * the Winograd weight gradient's range partials and the unfused Winograd
 * transforms of every conv call; plans shrink to fit, 0 means no such
 * scratch at all, and a split forced through MX_CONV_PLAN that does not fit
 * fails with MX_ERR_WORKSPACE. */
int mx_conv2d_plan(const mx_conv2d_desc* desc, int phase, int algo, int with_bias, mx_conv2d_plan_info* info);

/* Name of the main kernel a conv call with these arguments launches, e.g.
 * "conv_dw_kernel<64x64x32>": matches the kernel-trace names of a profiler and
 * keys per-kernel timing (the reference's gpu_timing_stats() per shader,
 * csrc/vulkan_context.cpp:368-404). */
int mx_conv2d_kernel_name(const mx_conv2d_desc* desc, int phase, int algo, char* buf, size_t len);

/* ------------------------------------------------------------------------ */
/* GEMM: mm / mm.out / addmm / bmm / bmm.out                                  */
/* ------------------------------------------------------------------------ */

enum mx_bias_kind { MX_BIAS_NONE = 0, MX_BIAS_COL = 1, MX_BIAS_MATRIX = 2 };

/* C[b] = alpha * A[b] x B[b] + beta * bias, with arbitrary element strides and
 * offsets for A and B (matmul_strided{,_reg}{,_bias}.comp, bmm_strided.comp;
 * mm_impl csrc/ops/mm.cpp:244-343, addmm_bias_vulkan :835-879, bmm_impl
 * csrc/ops/bmm.cpp:16-68).  C is written with row stride ldc and batch stride
 * batch_stride_c.  bias: MX_BIAS_COL = bias[n] (1-D addmm bias), MX_BIAS_MATRIX
 * = bias[m*bias_stride_m + n*bias_stride_n].  beta == 0 ignores the bias
 * entirely, NaN/Inf included (matmul_strided_reg_bias.comp:96).  k == 0 writes
 * beta*bias (or zeros). */
typedef struct mx_gemm_desc {
  int64_t batch, m, n, k;
  int64_t a_offset, a_stride_b, a_stride_m, a_stride_k;
  int64_t b_offset, b_stride_b, b_stride_k, b_stride_n;
  int64_t c_offset, c_stride_b, ldc;
  int64_t bias_offset, bias_stride_m, bias_stride_n;
  float alpha, beta;
  int bias_kind;
  int64_t bias_stride_b; /* bias batch stride (0 = one bias for every batch); ABI >= 2 */
  /* Tile family (ABI >= 3), the counterpart of TORCH_VULKAN_MM_KERNEL
   * (csrc/ops/mm.cpp:299-307, :851-854): MX_GEMM_KERNEL_AUTO lets the cost
   * model choose, MX_GEMM_KERNEL_TILED forces the small 64x64 tile (the
   * reference's 16x16 "tiled" kernel), MX_GEMM_KERNEL_REGISTER restricts the
   * choice to the large register-blocked tiles (its 64x64 "register" kernel). */
  int kernel;
} mx_gemm_desc;

enum mx_gemm_kernel { MX_GEMM_KERNEL_AUTO = 0, MX_GEMM_KERNEL_TILED = 1, MX_GEMM_KERNEL_REGISTER = 2 };

int mx_gemm_f32(const mx_gemm_desc* desc, const float* a, const float* b, const float* bias,
                float* c, void* stream);

/* Kernel instantiation mx_gemm_f32 launches for these arguments (tile,
 * operand loader modes, epilogue), e.g. "gemm_kernel<256x128x16,KVEC,RVEC>+bias_col";
 * a and b are only inspected for alignment.  The counterpart of the
 * reference's kernel choice in mm_impl (csrc/ops/mm.cpp:302-307). */
int mx_gemm_variant(const mx_gemm_desc* desc, const float* a, const float* b, char* buf, size_t len);

/* ------------------------------------------------------------------------ */
/* Multi-tensor fused AdamW                                                   */
/* ------------------------------------------------------------------------ */

/* One parameter tensor.  Either `step` (host, >= 1; bias corrections in double
 * on the host as csrc/ops/adamw.cpp:171-178) or `step_dev` (device FP32 scalar,
 * already incremented, as aten::_fused_adamw_'s state_steps) is used. */
typedef struct mx_adamw_tensor {
  float* param;
  float* grad;           /* read; written back unscaled when hparams.grad_scale is set */
  float* exp_avg;
  float* exp_avg_sq;
  float* max_exp_avg_sq; /* AMSGrad only, else NULL */
  int64_t numel;
  int64_t step;
  const float* step_dev;
} mx_adamw_tensor;

typedef struct mx_adamw_hparams {
  double lr, beta1, beta2, eps, weight_decay;
  int amsgrad;
  int maximize;
  const float* lr_dev;      /* optional device scalar lr (_fused_adamw_.tensor_lr) */
  const float* grad_scale;  /* optional device scalar: grads are divided by it and the unscaled
                            * grads written back (torch's fused AdamW under GradScaler) */
  const float* found_inf;   /* optional device scalar: when != 0 the step is skipped */
} mx_adamw_hparams;

/* Whole list in as few launches as the alias rule allows: entries that share a
 * written buffer with an earlier entry start a new launch, so repeated
 * parameters update sequentially (multitensor::partition conflict predicate,
 * csrc/ops/multitensor_plan.h:22-48, csrc/ops/adamw.cpp:207-215).
 * Replaces fused_adamw_step_ / fused_adamw_step_batch_impl
 * (csrc/ops/adamw.cpp:28-284) and adamw_fused{,_amsgrad}.comp /
 * adamw_multitensor{4,8}[_amsgrad].comp.  *launches (optional) receives the
 * number of kernel launches issued. */
int mx_adamw_step(const mx_adamw_tensor* tensors, int64_t count, const mx_adamw_hparams* hp,
                  int64_t* launches, void* stream);

/* ------------------------------------------------------------------------ */
/* Normalisation, activation, resampling, softmax, loss and concatenation   */
/* of the C3/C4 training steps (FP32, contiguous NCHW; rows r = n*C + c of  */
/* hw = H*W elements).  Results follow torch's CPU operators, the parity     */
/* target of the reference's kernels for the same ops.                       */
/* ------------------------------------------------------------------------ */

/* native_group_norm (csrc/ops/group_norm.cpp:73-107, group_norm_forward.comp):
 * y = (x - mean[n,g]) * rstd[n,g] * gamma[c] + beta[c]; mean / rstd are
 * [n, groups] (rstd = 1/sqrt(var + eps), biased variance).  gamma and beta may
 * be NULL (1 and 0).  n == 0 is a no-op. */
int mx_group_norm_forward(const float* x, const float* gamma, const float* beta, int64_t n, int64_t c,
                          int64_t hw, int64_t groups, float eps, float* y, float* mean, float* rstd,
                          void* stream);
/* native_group_norm_backward (csrc/ops/group_norm.cpp:109-153,
 * group_norm_backward_input.comp, group_norm_backward_affine.comp) from the
 * saved mean / rstd.  Any of dx, dgamma, dbeta may be NULL (not computed);
 * n == 0 writes zero dgamma / dbeta. */
int mx_group_norm_backward(const float* dy, const float* x, const float* mean, const float* rstd,
                           const float* gamma, int64_t n, int64_t c, int64_t hw, int64_t groups, float* dx,
                           float* dgamma, float* dbeta, void* stream);

/* native_batch_norm (csrc/ops/batch_norm.cpp:21-82, batch_norm_forward.comp).
 * training: batch statistics over (n, hw) per channel into save_mean /
 * save_invstd (invstd 0 when var == eps == 0), running statistics (element
 * strides rm_stride / rv_stride; NULL to skip) updated with momentum and the
 * unbiased variance.  evaluation: running statistics normalise.  gamma / beta
 * may be NULL. */
int mx_batch_norm_forward(const float* x, const float* gamma, const float* beta, float* running_mean,
                          int64_t rm_stride, float* running_var, int64_t rv_stride, int64_t n, int64_t c,
                          int64_t hw, int training, float momentum, float eps, float* y, float* save_mean,
                          float* save_invstd, void* stream);
/* native_batch_norm_backward (csrc/ops/batch_norm.cpp:83-110,
 * batch_norm_backward.comp).  training: `mean` / `invstd_or_var` are the saved
 * batch mean and inverse std; evaluation: the running mean and variance
 * (contiguous).  dx, dgamma, dbeta may be NULL. */
int mx_batch_norm_backward(const float* dy, const float* x, const float* gamma, const float* mean,
                           const float* invstd_or_var, int64_t n, int64_t c, int64_t hw, int training, float eps,
                           float* dx, float* dgamma, float* dbeta, void* stream);

/* Pointwise ops on `count` contiguous floats.  SiLU: x / (1 + exp(-x))
 * (csrc/ops/diffusion_unary.cpp:143, diffusion_unary.comp op 0); ReLU:
 * x <= 0 ? 0 : x, NaN kept (csrc/ops/mm.cpp:475-480). */
enum mx_unary_op { MX_UNARY_SILU = 0, MX_UNARY_RELU = 1 };
int mx_unary_f32(int op, const float* x, float* y, int64_t count, void* stream);
/* silu_backward: dy * s * (1 + x * (1 - s)), s = sigmoid(x)
 * (csrc/ops/diffusion_unary.cpp:151, diffusion_unary_backward.comp);
 * threshold_backward: x <= threshold ? 0 : dy (csrc/ops/mm.cpp:484-495). */
enum mx_unary_grad_op { MX_UNARY_SILU_GRAD = 0, MX_UNARY_THRESHOLD_GRAD = 1 };
int mx_unary_backward_f32(int op, const float* dy, const float* x, float threshold, float* dx,
                          int64_t count, void* stream);

/* upsample_nearest2d over `planes` = N*C planes (csrc/ops/upsample.cpp:7-45,
 * upsample_nearest2d.comp): source index = o for equal sizes, o >> 1 for
 * exact doubling, else min(floor(o * s), in - 1) with s = (float)(1/scale)
 * when scale > 0, else (float)in / out. */
int mx_upsample_nearest2d(const float* x, int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow,
                          double scale_h, double scale_w, float* y, void* stream);
/* upsample_nearest2d_backward (csrc/ops/upsample.cpp:46-56): each input pixel
 * sums the output gradients that read it, in row-major output order. */
int mx_upsample_nearest2d_backward(const float* dy, int64_t planes, int64_t ih, int64_t iw, int64_t oh,
                                   int64_t ow, double scale_h, double scale_w, float* dx, void* stream);

/* _softmax over the middle axis of a contiguous [outer, axis, inner] view
 * (csrc/ops/mm.cpp:1100, softmax_axis.comp): exp(x - max) * (1 / sum). */
int mx_softmax_f32(const float* x, int64_t outer, int64_t axis, int64_t inner, float* y, void* stream);
/* _softmax_backward_data (csrc/ops/softmax_axis_backward.cpp:11-38):
 * dx = y * (dy - sum(dy * y)). */
int mx_softmax_backward_f32(const float* dy, const float* y, int64_t outer, int64_t axis, int64_t inner,
                            float* dx, void* stream);

/* mse_loss (csrc/ops/loss_primitives.cpp:349-352): reduction NONE writes
 * (x - t)^2 elementwise, MEAN / SUM one float (mean of nothing is NaN). */
enum mx_reduction { MX_REDUCE_NONE = 0, MX_REDUCE_MEAN = 1, MX_REDUCE_SUM = 2 };
int mx_mse_loss_f32(const float* x, const float* t, int64_t count, int reduction, float* out, void* stream);
/* mse_loss_backward (csrc/ops/loss_primitives.cpp:353-356):
 * dx = norm * (x - t) * dy, norm = 2/count for MEAN else 2; dy is one device
 * float for MEAN / SUM and `count` floats for NONE. */
int mx_mse_loss_backward_f32(const float* dy, const float* x, const float* t, int64_t count, int reduction,
                             float* dx, void* stream);

/* Multi-tensor pointwise ops on contiguous FP32 tensors, one launch per list
 * (torch.optim's foreach path and the per-tensor lerp / addcmul / addcdiv /
 * maximum / minimum of csrc/ops/optimizer_primitives.cpp:12-202,
 * optimizer_pointwise.comp).  Entry i computes out[i] = f(a, b, c, scalar)
 * elementwise over numel elements (out may equal a: in place):
 *   MUL_SCALAR a*s   ADD_SCALAR a+s   DIV_SCALAR a/s   SQRT sqrt(a)
 *   LERP_SCALAR lerp(a, b, s)   LERP_TENSOR lerp(a, b, c)   (torch's two-branch lerp)
 *   ADDCMUL fma(s*b, c, a)   ADDCDIV a + (s*b)/c   ADD_LIST fma(b, s, a)
 *   MAXIMUM / MINIMUM of a and b (NaN propagates; a tie of signed zeros gives b).
 * Entries that write memory an earlier entry of the list touches start a new
 * launch, so repeated tensors update in list order.  *launches (optional)
 * receives the launch count. */
enum mx_foreach_op {
  MX_FOREACH_MUL_SCALAR = 0, MX_FOREACH_ADD_SCALAR = 1, MX_FOREACH_DIV_SCALAR = 2, MX_FOREACH_LERP_SCALAR = 3,
  MX_FOREACH_LERP_TENSOR = 4, MX_FOREACH_ADDCMUL = 5, MX_FOREACH_ADDCDIV = 6, MX_FOREACH_MAXIMUM = 7,
  MX_FOREACH_MINIMUM = 8, MX_FOREACH_SQRT = 9, MX_FOREACH_ADD_LIST = 10
};
typedef struct mx_foreach_tensor {
  float* out;
  const float* a;
  const float* b; /* NULL unless the op reads it */
  const float* c;
  int64_t numel;
  double scalar;
} mx_foreach_tensor;
int mx_foreach_f32(int op, const mx_foreach_tensor* tensors, int64_t count, int64_t* launches, void* stream);

/* Copy `rows` rows of `row_bytes` bytes between pitched buffers: one input's
 * slab of cat along any axis (csrc/ops/cat.cpp:44-55, cat_copy.comp). */
int mx_copy_rows(void* dst, int64_t dst_pitch, const void* src, int64_t src_pitch, int64_t row_bytes,
                 int64_t rows, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MX_H */
