/*
 * volta_hip.h -- C ABI of libvolta_hip.so, the MI355X (gfx950) implementation of
 * Volta's convolution and matrix-product hot path.
 *
 * Each compute entry point replaces one `RawTensor::gpu_*` function of the
 * reference's device-dispatch boundary (src/ops/gpu_ops.rs) or one CPU-only layer
 * routine of the same path, with the same argument meaning and order.  Cited
 * lines are under the reference root.
 *
 * Conventions
 *  - All pointers are device pointers (hipMalloc'd or torch-owned) except in
 *    vh_upload/vh_download.  Layouts are the reference's: NCHW activations,
 *    Conv2d weights OIHW (conv.rs:130), ConvTranspose2d weights IOHW
 *    (conv_transpose.rs:22,40), Linear weights [in, out] (linear.rs:9-10),
 *    row-major matrices.
 *  - `dtype` selects the storage type of every floating-point tensor argument of
 *    the call: VH_F32 (the reference's only type, storage.rs:583-585) or
 *    VH_BF16 (raw bf16 bits; the reference cannot compute in bf16).  Arithmetic
 *    always accumulates in fp32.  Bias vectors use the same dtype.
 *  - Outputs are written in full (no accumulation into existing contents).
 *  - `stream` is a hipStream_t (NULL = the default stream).  Calls are
 *    asynchronous with respect to the host; order is the stream's order.
 *  - Return value: VH_OK (0) or a vh_status code.  Where the reference returns
 *    Option::None (no device, CPU storage, allocation failure) this ABI returns
 *    a non-zero status so the caller keeps its CPU fallback; where the reference
 *    panics on a shape mismatch (kernels.rs:1129-1130) this ABI returns
 *    VH_ERR_BAD_SHAPE and never aborts the host.  vh_last_error() describes the
 *    last failure of the calling thread.
 *  - Every tensor must hold fewer than 2^31 elements (VH_ERR_UNSUPPORTED otherwise).
 *  - Workspace (split-K partials, re-laid-out weights, im2col matrices) is taken
 *    from one grow-only device buffer per stream inside the library; calls on
 *    one stream reuse it in stream order.  A HIP graph captured from library
 *    calls on a stream holds that stream's workspace address: its replays
 *    share the buffer with the capture stream's eager calls and with every
 *    other graph captured on that stream, wherever they are replayed, so such
 *    replays must be ordered with those calls and with each other (replay on
 *    the capture stream, or synchronise between them).  A buffer that a call
 *    outgrows is freed (after a synchronisation of its stream) when no
 *    captured call used it, and otherwise retired, so such a graph stays
 *    valid; retired and current workspaces are freed by vh_release_cache(),
 *    which therefore invalidates every such graph.  While a stream is being
 *    captured the library never allocates, frees or synchronises for it: a
 *    call whose workspace would have to grow returns VH_ERR_CAPTURE (run the
 *    call once eagerly on that stream before capturing).
 */
#ifndef VOLTA_HIP_H
#define VOLTA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  VH_OK = 0,
  VH_ERR_NO_DEVICE = 1,   /* no GPU: the reference's get_gpu_context() -> None */
  VH_ERR_BAD_SHAPE = 2,   /* dimension mismatch: the reference's assert_eq! panics */
  VH_ERR_OOM = 3,         /* device allocation failed: GpuBuffer::zeros -> None */
  VH_ERR_LAUNCH = 4,      /* HIP runtime / kernel launch error */
  VH_ERR_BAD_ARG = 5,     /* null pointer, bad enum value */
  VH_ERR_UNSUPPORTED = 6, /* tensor too large for 32-bit indexing; scratch maximum exceeded */
  VH_ERR_CAPTURE = 7      /* the stream's workspace would have to grow while the stream is
                             being captured into a HIP graph (see Workspace below) */
} vh_status;

typedef enum { VH_F32 = 0, VH_BF16 = 1 } vh_dtype;

/* ConvAlgo (src/nn/layers/conv.rs:11-24), same discriminant order. */
typedef enum { VH_ALGO_DIRECT = 0, VH_ALGO_IM2COL = 1, VH_ALGO_IGEMM = 2, VH_ALGO_AUTO = 3 } vh_conv_algo;

/* ------------------------------------------------------------------ runtime */
/* get_gpu_context (src/gpu/mod.rs:34-47): selects device 0 on first use. */
int vh_init(void);
const char* vh_last_error(void);
/* GpuBuffer::zeros / from_slice / to_vec (src/gpu/buffer.rs:40-220) and the
 * size-bucketed pool (src/gpu/pool.rs:28-35, 123-190).  Like the reference's
 * pool, which serves one in-order wgpu queue, the pool is single-stream: vh_free
 * makes the buffer available to the next vh_alloc at once, so free a buffer only
 * when every later use of the reallocated memory is ordered after its last use
 * (one stream, or a synchronisation in between). */
int vh_alloc(size_t bytes, void** dptr);
int vh_free(void* dptr);
int vh_upload(void* dst_dev, const void* src_host, size_t bytes, void* stream);
int vh_download(void* dst_host, const void* src_dev, size_t bytes, void* stream);
/* GpuContext::sync (src/gpu/context.rs:342-382). */
int vh_stream_sync(void* stream);
/* Releases cached workspace and pooled buffers (pool.rs clear) after a device
 * synchronisation.  Invalidates every HIP graph captured from library calls;
 * must not be called while a stream is being captured. */
int vh_release_cache(void);
/* Diagnostics (no reference counterpart): the current workspace of `stream`
 * (*ptr NULL and *bytes 0 when it has none yet) and how many outgrown
 * workspaces are kept because a call captured into a HIP graph used them.  Any
 * output pointer may be NULL. */
int vh_workspace_info(void* stream, void** ptr, size_t* bytes, size_t* retired);
/* Kernel choice inside an algorithm (no reference counterpart: Volta has one
 * shader per op).  VH_POLICY_FASTEST (default) uses specialised kernels where
 * their shape envelope allows; VH_POLICY_GENERIC forces the generic MFMA
 * implicit GEMM, so both can be checked against the same oracle. */
typedef enum { VH_POLICY_FASTEST = 0, VH_POLICY_GENERIC = 1 } vh_kernel_policy;
int vh_set_kernel_policy(int policy);

/* ------------------------------------------------------------------ matmul */
/* RawTensor::gpu_matmul, src/ops/gpu_ops.rs:151-169 (GpuKernels::matmul,
 * src/gpu/kernels.rs:1128-1210): c[m,n] = a[m,k] . b[k,n]. */
int vh_matmul(int dtype, const void* a, const void* b, void* c, int64_t m, int64_t k,
              int64_t n, void* stream);
/* RawTensor::gpu_matmul_backward_a, gpu_ops.rs:408-428 (kernels.rs:1218-1310):
 * grad_a[m,k] = grad[m,n] . b[k,n]^T. */
int vh_matmul_backward_a(int dtype, const void* grad, const void* b, void* grad_a,
                         int64_t m, int64_t k, int64_t n, void* stream);
/* RawTensor::gpu_matmul_backward_b, gpu_ops.rs:430-450 (kernels.rs:1318-1400):
 * grad_b[k,n] = a[m,k]^T . grad[m,n]. */
int vh_matmul_backward_b(int dtype, const void* a, const void* grad, void* grad_b,
                         int64_t m, int64_t k, int64_t n, void* stream);

/* ------------------------------------------------------------------ im2col */
/* RawTensor::gpu_im2col, gpu_ops.rs:515-544 (kernels.rs:2110-2215): input is the
 * already padded (B,C,H,W) tensor (conv.rs:1862-1879); col is
 * [B*h_out*w_out, C*kh*kw], row (b,oh,ow), column (c,kh,kw). */
int vh_im2col(int dtype, const void* input, void* col, int64_t batch, int64_t channels,
              int64_t height, int64_t width, int64_t kernel_h, int64_t kernel_w,
              int64_t stride_h, int64_t stride_w, int64_t h_out, int64_t w_out,
              void* stream);
/* RawTensor::gpu_col2im, gpu_ops.rs:546-572 (kernels.rs:2223-2310): adjoint of
 * vh_im2col (sum over every column entry that maps to an input element). */
int vh_col2im(int dtype, const void* col, void* output, int64_t batch, int64_t channels,
              int64_t height, int64_t width, int64_t kernel_h, int64_t kernel_w,
              int64_t stride_h, int64_t stride_w, int64_t h_out, int64_t w_out,
              void* stream);

/* ------------------------------------------------------------------ conv kernels */
/* Common dimension list, in the reference's order (stride BEFORE pad):
 * batch, in_channels, out_channels, height, width, kernel_h, kernel_w,
 * stride_h, stride_w, pad_h, pad_w, h_out, w_out.
 * h_out/w_out must equal (H + 2p - k)/s + 1, else VH_ERR_BAD_SHAPE. */

/* RawTensor::gpu_direct_conv, gpu_ops.rs:574-620 (kernels.rs:2318-2417,
 * direct_conv.wgsl:27-105): one output element per lane, fp32 accumulation. */
int vh_direct_conv(int dtype, const void* input, const void* weight, void* output,
                   int64_t batch, int64_t in_channels, int64_t out_channels, int64_t height,
                   int64_t width, int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                   int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t h_out,
                   int64_t w_out, void* stream);
/* RawTensor::gpu_igemm, gpu_ops.rs:622-668 (kernels.rs:2425-2536, igemm.wgsl):
 * implicit GEMM on MFMA (same math as vh_direct_conv). */
int vh_igemm(int dtype, const void* input, const void* weight, void* output, int64_t batch,
             int64_t in_channels, int64_t out_channels, int64_t height, int64_t width,
             int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w,
             int64_t pad_h, int64_t pad_w, int64_t h_out, int64_t w_out, void* stream);
/* RawTensor::gpu_conv_backward_input, gpu_ops.rs:670-716 (kernels.rs:2543-2640,
 * conv_backward_input.wgsl): grad_input (B,C,H,W) from out_grad and weight. */
int vh_conv_backward_input(int dtype, const void* out_grad, const void* weight,
                           void* grad_input, int64_t batch, int64_t in_channels,
                           int64_t out_channels, int64_t height, int64_t width,
                           int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                           int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t h_out,
                           int64_t w_out, void* stream);
/* RawTensor::gpu_conv_backward_weight, gpu_ops.rs:718-764 (kernels.rs:2647-2744,
 * conv_backward_weight.wgsl): grad_weight (O,C,KH,KW); note (out_grad, input). */
int vh_conv_backward_weight(int dtype, const void* out_grad, const void* input,
                            void* grad_weight, int64_t batch, int64_t in_channels,
                            int64_t out_channels, int64_t height, int64_t width,
                            int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                            int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t h_out,
                            int64_t w_out, void* stream);
/* RawTensor::gpu_igemm_backward_input, gpu_ops.rs:766-812 (kernels.rs:2750-2847). */
int vh_igemm_backward_input(int dtype, const void* out_grad, const void* weight,
                            void* grad_input, int64_t batch, int64_t in_channels,
                            int64_t out_channels, int64_t height, int64_t width,
                            int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                            int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t h_out,
                            int64_t w_out, void* stream);
/* RawTensor::gpu_igemm_backward_weight, gpu_ops.rs:814-861 (kernels.rs:2853-2950). */
int vh_igemm_backward_weight(int dtype, const void* out_grad, const void* input,
                             void* grad_weight, int64_t batch, int64_t in_channels,
                             int64_t out_channels, int64_t height, int64_t width,
                             int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                             int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t h_out,
                             int64_t w_out, void* stream);

/* ------------------------------------------------------------------ allocating forms */
/* The reference's gpu_* functions return a newly allocated result buffer
 * (GpuBuffer::zeros, src/gpu/kernels.rs:1133,1233,1333; wrapped as Storage::Gpu,
 * src/ops/gpu_ops.rs:160-168).  Each *_alloc takes the output from the
 * library's pool (release it with vh_free), runs the entry point above into it
 * and returns it in *out (NULL on failure); same arguments otherwise. */
int vh_matmul_alloc(int dtype, const void* a, const void* b, void** c, int64_t m, int64_t k,
                    int64_t n, void* stream);                        /* gpu_ops.rs:151 */
int vh_matmul_backward_a_alloc(int dtype, const void* grad, const void* b, void** grad_a,
                               int64_t m, int64_t k, int64_t n, void* stream); /* gpu_ops.rs:408 */
int vh_matmul_backward_b_alloc(int dtype, const void* a, const void* grad, void** grad_b,
                               int64_t m, int64_t k, int64_t n, void* stream); /* gpu_ops.rs:430 */
int vh_im2col_alloc(int dtype, const void* input, void** col, int64_t batch, int64_t channels,
                    int64_t height, int64_t width, int64_t kernel_h, int64_t kernel_w,
                    int64_t stride_h, int64_t stride_w, int64_t h_out, int64_t w_out,
                    void* stream);                                    /* gpu_ops.rs:515 */
int vh_col2im_alloc(int dtype, const void* col, void** output, int64_t batch, int64_t channels,
                    int64_t height, int64_t width, int64_t kernel_h, int64_t kernel_w,
                    int64_t stride_h, int64_t stride_w, int64_t h_out, int64_t w_out,
                    void* stream);                                    /* gpu_ops.rs:546 */
/* Conv forms: (t0, t1) are the two inputs of the out-parameter entry point in its
 * order -- (input, weight), (out_grad, weight) or (out_grad, input). */
int vh_direct_conv_alloc(int dtype, const void* t0, const void* t1, void** out, int64_t batch,
                         int64_t in_channels, int64_t out_channels, int64_t height, int64_t width,
                         int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w,
                         int64_t pad_h, int64_t pad_w, int64_t h_out, int64_t w_out,
                         void* stream);                               /* gpu_ops.rs:574 */
int vh_igemm_alloc(int dtype, const void* t0, const void* t1, void** out, int64_t batch,
                   int64_t in_channels, int64_t out_channels, int64_t height, int64_t width,
                   int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w,
                   int64_t pad_h, int64_t pad_w, int64_t h_out, int64_t w_out,
                   void* stream);                                     /* gpu_ops.rs:622 */
int vh_conv_backward_input_alloc(int dtype, const void* t0, const void* t1, void** out,
                                 int64_t batch, int64_t in_channels, int64_t out_channels,
                                 int64_t height, int64_t width, int64_t kernel_h, int64_t kernel_w,
                                 int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                                 int64_t h_out, int64_t w_out, void* stream); /* gpu_ops.rs:670 */
int vh_igemm_backward_input_alloc(int dtype, const void* t0, const void* t1, void** out,
                                  int64_t batch, int64_t in_channels, int64_t out_channels,
                                  int64_t height, int64_t width, int64_t kernel_h, int64_t kernel_w,
                                  int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                                  int64_t h_out, int64_t w_out, void* stream); /* gpu_ops.rs:766 */
int vh_conv_backward_weight_alloc(int dtype, const void* t0, const void* t1, void** out,
                                  int64_t batch, int64_t in_channels, int64_t out_channels,
                                  int64_t height, int64_t width, int64_t kernel_h, int64_t kernel_w,
                                  int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                                  int64_t h_out, int64_t w_out, void* stream); /* gpu_ops.rs:718 */
int vh_igemm_backward_weight_alloc(int dtype, const void* t0, const void* t1, void** out,
                                   int64_t batch, int64_t in_channels, int64_t out_channels,
                                   int64_t height, int64_t width, int64_t kernel_h, int64_t kernel_w,
                                   int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                                   int64_t h_out, int64_t w_out, void* stream); /* gpu_ops.rs:814 */

/* ------------------------------------------------------------------ layers */
/* ConvAlgo::auto_select, conv.rs:29-69, verbatim rule (both branches); returns
 * the vh_conv_algo value, or -1 if height/width < kernel_size. */
int vh_conv_algo_auto_select(int64_t batch, int64_t channels, int64_t height, int64_t width,
                             int64_t kernel_size, int has_gpu);
/* The selector this library applies for VH_ALGO_AUTO on MI355X (same inputs as
 * conv.rs:1821-1832 plus the full geometry); returns DIRECT, IM2COL or IGEMM. */
int vh_conv_algo_select_mi355x(int64_t batch, int64_t in_channels, int64_t out_channels,
                               int64_t height, int64_t width, int64_t kernel_h,
                               int64_t kernel_w, int64_t stride_h, int64_t stride_w,
                               int64_t pad_h, int64_t pad_w);

/* Conv2d::forward, conv.rs:1787-1927: algorithm dispatch (algo may be AUTO) and
 * the bias add of conv.rs:1915-1926 (bias may be NULL). *algo_used receives the
 * algorithm that ran (may be NULL).  Dimensions as above without h_out/w_out. */
int vh_conv2d_forward(int dtype, int algo, const void* input, const void* weight,
                      const void* bias, void* output, int64_t batch, int64_t in_channels,
                      int64_t out_channels, int64_t height, int64_t width, int64_t kernel_h,
                      int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                      int64_t pad_w, int* algo_used, void* stream);
/* Backward of Conv2d::forward: DirectConvGradFn (conv.rs:216-414),
 * Im2colGradFn + MatMulGradFn (conv.rs:139-208, matmul.rs:378-460),
 * IGEMMGradFn (conv.rs:617-768), bias grad via expand backward
 * (movement.rs:441-485).  Any of grad_input / grad_weight / grad_bias may be
 * NULL to skip it.  algo must be the algorithm the forward used (not AUTO). */
int vh_conv2d_backward(int dtype, int algo, const void* out_grad, const void* input,
                       const void* weight, void* grad_input, void* grad_weight,
                       void* grad_bias, int64_t batch, int64_t in_channels,
                       int64_t out_channels, int64_t height, int64_t width, int64_t kernel_h,
                       int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                       int64_t pad_w, void* stream);

/* ConvTranspose2d forward, conv_transpose.rs:356-435 (CPU-only in the
 * reference): weight IOHW [in, out, kh, kw], bias may be NULL, output
 * (B, out, (H-1)s+kh-2p, (W-1)s+kw-2p). */
int vh_conv_transpose2d_forward(int dtype, const void* input, const void* weight,
                                const void* bias, void* output, int64_t batch,
                                int64_t in_channels, int64_t out_channels, int64_t height,
                                int64_t width, int64_t kernel_h, int64_t kernel_w,
                                int64_t stride_h, int64_t stride_w, int64_t pad_h,
                                int64_t pad_w, void* stream);
/* ConvTranspose2dGradFn::backward, conv_transpose.rs:161-341; NULL skips. */
int vh_conv_transpose2d_backward(int dtype, const void* out_grad, const void* input,
                                 const void* weight, void* grad_input, void* grad_weight,
                                 void* grad_bias, int64_t batch, int64_t in_channels,
                                 int64_t out_channels, int64_t height, int64_t width,
                                 int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                                 int64_t stride_w, int64_t pad_h, int64_t pad_w,
                                 void* stream);

/* Linear::forward, linear.rs:110-117: y[m,out] = x[m,in] . w[in,out] + bias
 * (bias may be NULL). */
int vh_linear_forward(int dtype, const void* x, const void* weight, const void* bias, void* y,
                      int64_t m, int64_t in_features, int64_t out_features, void* stream);
/* Linear backward: MatMulGradFn (matmul.rs:389-444) + BinaryGradFn bias
 * reduction (binary.rs:533-598); NULL skips an output. */
int vh_linear_backward(int dtype, const void* out_grad, const void* x, const void* weight,
                       void* grad_x, void* grad_weight, void* grad_bias, int64_t m,
                       int64_t in_features, int64_t out_features, void* stream);

/* PixelShuffle::forward, pixelshuffle.rs:50-85: (B, C*r*r, H, W) -> (B, C, H*r, W*r);
 * `channels` is the OUTPUT channel count C. */
int vh_pixel_shuffle(int dtype, const void* input, void* output, int64_t batch,
                     int64_t channels, int64_t height, int64_t width, int64_t upscale,
                     void* stream);
/* Backward: the inverse permutation (movement.rs:407-440). */
int vh_pixel_shuffle_backward(int dtype, const void* out_grad, void* grad_input,
                              int64_t batch, int64_t channels, int64_t height, int64_t width,
                              int64_t upscale, void* stream);

/* Fused forms for the config graphs' conv -> ReLU chains (no single counterpart in
 * the reference, which runs Conv2d::forward then relu, and ReLU's backward after the
 * next layer's input gradient; same results):
 * vh_conv2d_forward_relu = vh_conv2d_forward followed by ReLU (unary.rs:272), the
 * ReLU applied in the convolution's epilogue; */
int vh_conv2d_forward_relu(int dtype, int algo, const void* input, const void* weight,
                           const void* bias, void* output, int64_t batch, int64_t in_channels,
                           int64_t out_channels, int64_t height, int64_t width, int64_t kernel_h,
                           int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                           int64_t pad_w, int* algo_used, void* stream);
/* vh_conv2d_backward_relu = vh_conv2d_backward for a layer whose input came out of a
 * ReLU, with that ReLU's backward (unary.rs:150-155) applied to grad_input:
 * grad_input = input > 0 ? dX : 0 (the ReLU's output is positive exactly where its
 * input was), in the input-gradient epilogue. */
int vh_conv2d_backward_relu(int dtype, int algo, const void* out_grad, const void* input,
                            const void* weight, void* grad_input, void* grad_weight, void* grad_bias,
                            int64_t batch, int64_t in_channels, int64_t out_channels, int64_t height,
                            int64_t width, int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                            int64_t stride_w, int64_t pad_h, int64_t pad_w, void* stream);

/* Allocation-free variant of vh_conv2d_backward (no counterpart in the reference):
 * for callers that cannot allocate device memory -- code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc.  Same arguments, algorithms,
 * kernels and results as vh_conv2d_backward; its workspace (re-laid-out weights,
 * split-K partial sums, im2col matrices) is a static device array of
 * VH_NOALLOC_SCRATCH_BYTES per GPU, held from the library's first use on that GPU
 * until the process ends.  The call never allocates or frees: a call that would
 * need more workspace returns VH_ERR_UNSUPPORTED before anything is queued.  Every
 * call on one GPU shares that GPU's array, so calls that overlap on one GPU (two
 * streams, two threads, without ordering between them) race; order them. */
#define VH_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int vh_conv2d_backward_noalloc(int dtype, int algo, const void* out_grad, const void* input,
                               const void* weight, void* grad_input, void* grad_weight,
                               void* grad_bias, int64_t batch, int64_t in_channels,
                               int64_t out_channels, int64_t height, int64_t width,
                               int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                               int64_t stride_w, int64_t pad_h, int64_t pad_w, void* stream);

/* ---- Glue of the config graphs (ReLU between layers, the sum loss, its seed) ---- */
#define VH_UNARY_RELU 0
/* gpu_ops.rs:171 gpu_unary(input, "relu") (unary.rs:272): y = max(x, 0), NaN -> 0.
 * Only VH_UNARY_RELU is on this path; other ops return VH_ERR_UNSUPPORTED. */
int vh_unary(int dtype, int op, const void* input, void* output, int64_t n, void* stream);
/* gpu_ops.rs:186 gpu_unary_backward(out_grad, x, "relu") (unary.rs:150-155):
 * grad_input = x > 0 ? out_grad : 0, with x the forward input. */
int vh_unary_backward(int dtype, int op, const void* out_grad, const void* input, void* grad_input,
                      int64_t n, void* stream);
/* gpu_ops.rs:118 gpu_sum_reduce (ReduceOp::Sum, reduce.rs:160-180): the fp32 sum of
 * the n elements, written to `result` (one float in device memory; the reference
 * returns it to the host).  Fixed summation order for a given n. */
int vh_sum_reduce(int dtype, const void* input, int64_t n, float* result, void* stream);
/* gpu_ops.rs:452 gpu_sum_backward(grad, size) (SumGradFn, reduce.rs:22-45): every
 * element = grad (rounded to dtype).  With grad = 1 it is the autograd seed
 * (autograd.rs:49-62). */
int vh_sum_backward(int dtype, float grad, void* grad_input, int64_t n, void* stream);

/* ---- Device storage: dtype and layout (the reference keeps device data f32 and
 * NCHW, storage.rs:570-597; these let it stay bf16 and convert layouts on the GPU) ---- */
/* n elements: bf16 -> f32 exact, f32 -> bf16 round-to-nearest-even (as half::bf16::from_f32,
 * storage.rs:503-505); equal dtypes copy. */
int vh_cast(int src_dtype, int dst_dtype, const void* src, void* dst, int64_t n, void* stream);
/* [B][C][H][W] <-> [B][H][W][C]; src and dst must not overlap. */
int vh_nchw_to_nhwc(int dtype, const void* src, void* dst, int64_t batch, int64_t channels,
                    int64_t height, int64_t width, void* stream);
int vh_nhwc_to_nchw(int dtype, const void* src, void* dst, int64_t batch, int64_t channels,
                    int64_t height, int64_t width, void* stream);

/* ---- The step after the weight gradient ---- */
/* autograd.rs:158-184 accumulate_grad (gpu_add, gpu_ops.rs:17): existing += new_grad,
 * in place (the reference allocates the sum and drops the old buffer). */
int vh_grad_accumulate(int dtype, void* existing, const void* new_grad, int64_t n, void* stream);
#define VH_OPT_SGD 0
#define VH_OPT_SGD_MOMENTUM 1
#define VH_OPT_ADAM 2
/* gpu_ops.rs:496 gpu_optimizer_step (optimizer_step.wgsl; SGD::step's GPU path,
 * sgd.rs:94-180): one update of n f32 parameters in place.  g = grad (+ weight_decay *
 * param); SGD: param -= lr*g; momentum: s1 = beta1*s1 - lr*g, param += s1 (s1 = the
 * velocity); Adam: s1/s2 = first/second moments, bias correction with step t.
 * state1 may be NULL for op 0, state2 for ops 0 and 1. */
int vh_optimizer_step(int op, float lr, float beta1, float beta2, float t, float eps,
                      float weight_decay, float* params, const float* grads, float* state1,
                      float* state2, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* VOLTA_HIP_H */
