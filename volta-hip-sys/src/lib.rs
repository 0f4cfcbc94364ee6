//! Raw FFI declarations of `libvolta_hip.so` (`include/volta_hip.h`), the
//! MI355X implementation of Volta's convolution / matrix-product path.
//!
//! One `extern "C"` declaration per function of the header, in header order;
//! `tests/test_rust_ffi.py` checks names, parameter counts and types against
//! the header.  Device pointers are `*const c_void` / `*mut c_void`, sizes
//! `i64`, streams `*mut c_void` (a `hipStream_t`; null = default stream), and
//! every function returns a status (`VH_OK` = 0).  The safe layer Volta calls
//! from `src/ops/gpu_ops.rs` is the [`gpu_ops`] module: an owned device buffer
//! and one `gpu_*` function per conv / matmul entry of the reference's
//! `gpu_ops.rs`, where a non-zero status becomes `None`, keeping the CPU
//! fallback.
#![allow(non_camel_case_types)]
use std::ffi::{c_char, c_int, c_void, CStr};

pub mod gpu_ops;

pub const VH_OK: c_int = 0;
pub const VH_ERR_NO_DEVICE: c_int = 1;
pub const VH_ERR_BAD_SHAPE: c_int = 2;
pub const VH_ERR_OOM: c_int = 3;
pub const VH_ERR_LAUNCH: c_int = 4;
pub const VH_ERR_BAD_ARG: c_int = 5;
pub const VH_ERR_UNSUPPORTED: c_int = 6;
pub const VH_ERR_CAPTURE: c_int = 7;

pub const VH_F32: c_int = 0;
pub const VH_BF16: c_int = 1;

/// `ConvAlgo` (src/nn/layers/conv.rs:11-24), same discriminants.
pub const VH_ALGO_DIRECT: c_int = 0;
pub const VH_ALGO_IM2COL: c_int = 1;
pub const VH_ALGO_IGEMM: c_int = 2;
pub const VH_ALGO_AUTO: c_int = 3;

pub const VH_POLICY_FASTEST: c_int = 0;
pub const VH_POLICY_GENERIC: c_int = 1;
pub const VH_UNARY_RELU: c_int = 0;
pub const VH_OPT_SGD: c_int = 0;
pub const VH_OPT_SGD_MOMENTUM: c_int = 1;
pub const VH_OPT_ADAM: c_int = 2;
/// Static scratch of `vh_conv2d_backward_noalloc` per GPU (bytes).
pub const VH_NOALLOC_SCRATCH_BYTES: usize = 64 << 20;

extern "C" {
    pub fn vh_init() -> c_int;
    pub fn vh_last_error() -> *const c_char;
    pub fn vh_alloc(bytes: usize, dptr: *mut *mut c_void) -> c_int;
    pub fn vh_free(dptr: *mut c_void) -> c_int;
    pub fn vh_upload(dst_dev: *mut c_void, src_host: *const c_void, bytes: usize, stream: *mut c_void) -> c_int;
    pub fn vh_download(dst_host: *mut c_void, src_dev: *const c_void, bytes: usize, stream: *mut c_void) -> c_int;
    pub fn vh_stream_sync(stream: *mut c_void) -> c_int;
    pub fn vh_release_cache() -> c_int;
    pub fn vh_workspace_info(stream: *mut c_void, ptr: *mut *mut c_void, bytes: *mut usize, retired: *mut usize) -> c_int;
    pub fn vh_set_kernel_policy(policy: c_int) -> c_int;
    pub fn vh_matmul(dtype: c_int, a: *const c_void, b: *const c_void, c: *mut c_void, m: i64, k: i64, n: i64, stream: *mut c_void) -> c_int;
    pub fn vh_matmul_backward_a(dtype: c_int, grad: *const c_void, b: *const c_void, grad_a: *mut c_void, m: i64, k: i64, n: i64, stream: *mut c_void) -> c_int;
    pub fn vh_matmul_backward_b(dtype: c_int, a: *const c_void, grad: *const c_void, grad_b: *mut c_void, m: i64, k: i64, n: i64, stream: *mut c_void) -> c_int;
    pub fn vh_im2col(dtype: c_int, input: *const c_void, col: *mut c_void, batch: i64, channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_col2im(dtype: c_int, col: *const c_void, output: *mut c_void, batch: i64, channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_direct_conv(dtype: c_int, input: *const c_void, weight: *const c_void, output: *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_igemm(dtype: c_int, input: *const c_void, weight: *const c_void, output: *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_conv_backward_input(dtype: c_int, out_grad: *const c_void, weight: *const c_void, grad_input: *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_conv_backward_weight(dtype: c_int, out_grad: *const c_void, input: *const c_void, grad_weight: *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_igemm_backward_input(dtype: c_int, out_grad: *const c_void, weight: *const c_void, grad_input: *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_igemm_backward_weight(dtype: c_int, out_grad: *const c_void, input: *const c_void, grad_weight: *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_matmul_alloc(dtype: c_int, a: *const c_void, b: *const c_void, c: *mut *mut c_void, m: i64, k: i64, n: i64, stream: *mut c_void) -> c_int;
    pub fn vh_matmul_backward_a_alloc(dtype: c_int, grad: *const c_void, b: *const c_void, grad_a: *mut *mut c_void, m: i64, k: i64, n: i64, stream: *mut c_void) -> c_int;
    pub fn vh_matmul_backward_b_alloc(dtype: c_int, a: *const c_void, grad: *const c_void, grad_b: *mut *mut c_void, m: i64, k: i64, n: i64, stream: *mut c_void) -> c_int;
    pub fn vh_im2col_alloc(dtype: c_int, input: *const c_void, col: *mut *mut c_void, batch: i64, channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_col2im_alloc(dtype: c_int, col: *const c_void, output: *mut *mut c_void, batch: i64, channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_direct_conv_alloc(dtype: c_int, t0: *const c_void, t1: *const c_void, out: *mut *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_igemm_alloc(dtype: c_int, t0: *const c_void, t1: *const c_void, out: *mut *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_conv_backward_input_alloc(dtype: c_int, t0: *const c_void, t1: *const c_void, out: *mut *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_igemm_backward_input_alloc(dtype: c_int, t0: *const c_void, t1: *const c_void, out: *mut *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_conv_backward_weight_alloc(dtype: c_int, t0: *const c_void, t1: *const c_void, out: *mut *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_igemm_backward_weight_alloc(dtype: c_int, t0: *const c_void, t1: *const c_void, out: *mut *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, h_out: i64, w_out: i64, stream: *mut c_void) -> c_int;
    pub fn vh_conv_algo_auto_select(batch: i64, channels: i64, height: i64, width: i64, kernel_size: i64, has_gpu: c_int) -> c_int;
    pub fn vh_conv_algo_select_mi355x(batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64) -> c_int;
    pub fn vh_conv2d_forward(dtype: c_int, algo: c_int, input: *const c_void, weight: *const c_void, bias: *const c_void, output: *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, algo_used: *mut c_int, stream: *mut c_void) -> c_int;
    pub fn vh_conv2d_backward(dtype: c_int, algo: c_int, out_grad: *const c_void, input: *const c_void, weight: *const c_void, grad_input: *mut c_void, grad_weight: *mut c_void, grad_bias: *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, stream: *mut c_void) -> c_int;
    pub fn vh_conv_transpose2d_forward(dtype: c_int, input: *const c_void, weight: *const c_void, bias: *const c_void, output: *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, stream: *mut c_void) -> c_int;
    pub fn vh_conv_transpose2d_backward(dtype: c_int, out_grad: *const c_void, input: *const c_void, weight: *const c_void, grad_input: *mut c_void, grad_weight: *mut c_void, grad_bias: *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, stream: *mut c_void) -> c_int;
    pub fn vh_linear_forward(dtype: c_int, x: *const c_void, weight: *const c_void, bias: *const c_void, y: *mut c_void, m: i64, in_features: i64, out_features: i64, stream: *mut c_void) -> c_int;
    pub fn vh_linear_backward(dtype: c_int, out_grad: *const c_void, x: *const c_void, weight: *const c_void, grad_x: *mut c_void, grad_weight: *mut c_void, grad_bias: *mut c_void, m: i64, in_features: i64, out_features: i64, stream: *mut c_void) -> c_int;
    pub fn vh_pixel_shuffle(dtype: c_int, input: *const c_void, output: *mut c_void, batch: i64, channels: i64, height: i64, width: i64, upscale: i64, stream: *mut c_void) -> c_int;
    pub fn vh_pixel_shuffle_backward(dtype: c_int, out_grad: *const c_void, grad_input: *mut c_void, batch: i64, channels: i64, height: i64, width: i64, upscale: i64, stream: *mut c_void) -> c_int;
    pub fn vh_conv2d_forward_relu(dtype: c_int, algo: c_int, input: *const c_void, weight: *const c_void, bias: *const c_void, output: *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, algo_used: *mut c_int, stream: *mut c_void) -> c_int;
    pub fn vh_conv2d_backward_relu(dtype: c_int, algo: c_int, out_grad: *const c_void, input: *const c_void, weight: *const c_void, grad_input: *mut c_void, grad_weight: *mut c_void, grad_bias: *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, stream: *mut c_void) -> c_int;
    pub fn vh_conv2d_backward_noalloc(dtype: c_int, algo: c_int, out_grad: *const c_void, input: *const c_void, weight: *const c_void, grad_input: *mut c_void, grad_weight: *mut c_void, grad_bias: *mut c_void, batch: i64, in_channels: i64, out_channels: i64, height: i64, width: i64, kernel_h: i64, kernel_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64, stream: *mut c_void) -> c_int;
    pub fn vh_unary(dtype: c_int, op: c_int, input: *const c_void, output: *mut c_void, n: i64, stream: *mut c_void) -> c_int;
    pub fn vh_unary_backward(dtype: c_int, op: c_int, out_grad: *const c_void, input: *const c_void, grad_input: *mut c_void, n: i64, stream: *mut c_void) -> c_int;
    pub fn vh_sum_reduce(dtype: c_int, input: *const c_void, n: i64, result: *mut f32, stream: *mut c_void) -> c_int;
    pub fn vh_sum_backward(dtype: c_int, grad: f32, grad_input: *mut c_void, n: i64, stream: *mut c_void) -> c_int;
    pub fn vh_cast(src_dtype: c_int, dst_dtype: c_int, src: *const c_void, dst: *mut c_void, n: i64, stream: *mut c_void) -> c_int;
    pub fn vh_nchw_to_nhwc(dtype: c_int, src: *const c_void, dst: *mut c_void, batch: i64, channels: i64, height: i64, width: i64, stream: *mut c_void) -> c_int;
    pub fn vh_nhwc_to_nchw(dtype: c_int, src: *const c_void, dst: *mut c_void, batch: i64, channels: i64, height: i64, width: i64, stream: *mut c_void) -> c_int;
    pub fn vh_grad_accumulate(dtype: c_int, existing: *mut c_void, new_grad: *const c_void, n: i64, stream: *mut c_void) -> c_int;
    pub fn vh_optimizer_step(op: c_int, lr: f32, beta1: f32, beta2: f32, t: f32, eps: f32, weight_decay: f32, params: *mut f32, grads: *const f32, state1: *mut f32, state2: *mut f32, n: i64, stream: *mut c_void) -> c_int;

}

/// A failed call: the status and `vh_last_error()`'s message.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct Error {
    pub status: c_int,
    pub message: String,
}

/// `Ok(())` for `VH_OK`, else the status with the library's message.
pub fn check(status: c_int) -> Result<(), Error> {
    if status == VH_OK {
        return Ok(());
    }
    // SAFETY: vh_last_error returns a NUL-terminated thread-local buffer.
    let message = unsafe { CStr::from_ptr(vh_last_error()) }.to_string_lossy().into_owned();
    Err(Error { status, message })
}
