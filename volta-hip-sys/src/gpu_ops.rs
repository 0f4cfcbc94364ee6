//! Safe layer over the raw declarations: the `RawTensor::gpu_*` functions of
//! Volta's `src/ops/gpu_ops.rs` on the convolution / matrix-product path (plus
//! the ReLU, sum-loss and seed glue of the config graphs), with the
//! reference's names, parameter names, parameter order and `usize`
//! dimensions.  Each body converts the dimensions, calls one `extern "C"`
//! function and maps a non-zero status to `None`, so Volta's callers keep
//! their CPU fallback (`conv.rs:696-731, 773-806, 1509-1511`, `matmul.rs:187`).
//!
//! [`DeviceBuffer`] stands where Volta's `Storage::Gpu { buffer: Arc<GpuBuffer>, .. }`
//! does (`gpu_ops.rs:160-168`): device memory from the library's pool
//! (`vh_alloc`), returned to it when dropped, as a `GpuBuffer` returns to
//! `pool.rs` (`src/gpu/buffer.rs:289-300`).  It also carries the element
//! type (`VH_F32` or `VH_BF16`); both operands of a call must share it.
//! Calls run on the default HIP stream in issue order, like Volta's single
//! wgpu queue; reading a buffer back synchronises.
use std::ffi::{c_int, c_void};
use std::ptr;

use crate::*;

/// The stream of every call of this layer: the default stream (in order).
const STREAM: *mut c_void = ptr::null_mut();

/// Bytes per element of a `vh_dtype`.
fn elem_size(dtype: c_int) -> Option<usize> {
    match dtype {
        VH_F32 => Some(4),
        VH_BF16 => Some(2),
        _ => None,
    }
}

/// A dimension as the ABI's `int64_t` (`None` if it does not fit).
fn dim(x: usize) -> Option<i64> {
    i64::try_from(x).ok()
}

/// Product of element counts (`None` on overflow).
fn count(dims: &[usize]) -> Option<usize> {
    dims.iter().try_fold(1usize, |acc, &d| acc.checked_mul(d))
}

/// Device memory of `len` elements of one dtype, owned; freed into the
/// library's pool on drop.
#[derive(Debug)]
pub struct DeviceBuffer {
    ptr: *mut c_void,
    len: usize,
    dtype: c_int,
}

// SAFETY: the pointer is device memory owned by this value alone; the pool
// behind vh_alloc / vh_free is guarded by a mutex inside the library.
unsafe impl Send for DeviceBuffer {}
unsafe impl Sync for DeviceBuffer {}

impl DeviceBuffer {
    /// Uninitialised device memory for `len` elements (`GpuBuffer::new`,
    /// `src/gpu/buffer.rs:40-60`).
    pub fn new(len: usize, dtype: c_int) -> Option<DeviceBuffer> {
        let bytes = len.checked_mul(elem_size(dtype)?)?;
        let mut p: *mut c_void = ptr::null_mut();
        // SAFETY: `p` is a valid out-pointer for the allocation.
        check(unsafe { vh_alloc(bytes, &mut p) }).ok()?;
        Some(DeviceBuffer { ptr: p, len, dtype })
    }

    /// An f32 buffer holding `data` (`GpuBuffer::from_slice`, `src/gpu/buffer.rs:62-95`).
    pub fn from_f32(data: &[f32]) -> Option<DeviceBuffer> {
        let buf = DeviceBuffer::new(data.len(), VH_F32)?;
        // SAFETY: `buf` holds `data.len()` f32 elements; the source is a live slice.
        check(unsafe { vh_upload(buf.ptr, data.as_ptr() as *const c_void, buf.bytes(), STREAM) }).ok()?;
        Some(buf)
    }

    /// A bf16 buffer from bf16 bit patterns (what `Storage::to_dtype(BF16)`
    /// holds, `src/storage.rs:503-505`).
    pub fn from_bf16_bits(data: &[u16]) -> Option<DeviceBuffer> {
        let buf = DeviceBuffer::new(data.len(), VH_BF16)?;
        // SAFETY: `buf` holds `data.len()` bf16 elements; the source is a live slice.
        check(unsafe { vh_upload(buf.ptr, data.as_ptr() as *const c_void, buf.bytes(), STREAM) }).ok()?;
        Some(buf)
    }

    /// The contents of an f32 buffer (`GpuBuffer::to_vec`, `src/gpu/buffer.rs:137-220`).
    pub fn to_f32_vec(&self) -> Option<Vec<f32>> {
        if self.dtype != VH_F32 {
            return None;
        }
        let mut out = vec![0.0f32; self.len];
        // SAFETY: `out` has room for `self.len` f32 elements.
        check(unsafe { vh_download(out.as_mut_ptr() as *mut c_void, self.ptr, self.bytes(), STREAM) }).ok()?;
        Some(out)
    }

    /// The bit patterns of a bf16 buffer.
    pub fn to_bf16_bits(&self) -> Option<Vec<u16>> {
        if self.dtype != VH_BF16 {
            return None;
        }
        let mut out = vec![0u16; self.len];
        // SAFETY: `out` has room for `self.len` bf16 elements.
        check(unsafe { vh_download(out.as_mut_ptr() as *mut c_void, self.ptr, self.bytes(), STREAM) }).ok()?;
        Some(out)
    }

    pub fn len(&self) -> usize {
        self.len
    }

    pub fn is_empty(&self) -> bool {
        self.len == 0
    }

    pub fn dtype(&self) -> c_int {
        self.dtype
    }

    pub fn bytes(&self) -> usize {
        self.len * elem_size(self.dtype).unwrap_or(0)
    }

    pub fn as_ptr(&self) -> *const c_void {
        self.ptr
    }

    pub fn as_mut_ptr(&mut self) -> *mut c_void {
        self.ptr
    }
}

impl Drop for DeviceBuffer {
    fn drop(&mut self) {
        // SAFETY: `ptr` came from vh_alloc (directly or through an *_alloc
        // entry point) and is released exactly once.
        unsafe {
            vh_free(self.ptr);
        }
    }
}

/// The shared dtype of two operands (`None` if they differ).
fn same_dtype(a: &DeviceBuffer, b: &DeviceBuffer) -> Option<c_int> {
    if a.dtype == b.dtype {
        Some(a.dtype)
    } else {
        None
    }
}

/// Runs an allocating entry point and takes ownership of its output of `len`
/// elements; `None` on a non-zero status.
fn alloc_out<F>(len: usize, dtype: c_int, call: F) -> Option<DeviceBuffer>
where
    F: FnOnce(*mut *mut c_void) -> c_int,
{
    let mut out: *mut c_void = ptr::null_mut();
    let status = call(&mut out);
    if status != VH_OK || out.is_null() {
        return None;
    }
    Some(DeviceBuffer { ptr: out, len, dtype })
}

/// The 13 dimensions of a convolution call as the ABI's `int64_t`.
#[allow(clippy::too_many_arguments)]
fn conv_dims(
    batch_size: usize,
    in_channels: usize,
    out_channels: usize,
    height: usize,
    width: usize,
    kernel_h: usize,
    kernel_w: usize,
    stride_h: usize,
    stride_w: usize,
    pad_h: usize,
    pad_w: usize,
    h_out: usize,
    w_out: usize,
) -> Option<[i64; 13]> {
    Some([
        dim(batch_size)?,
        dim(in_channels)?,
        dim(out_channels)?,
        dim(height)?,
        dim(width)?,
        dim(kernel_h)?,
        dim(kernel_w)?,
        dim(stride_h)?,
        dim(stride_w)?,
        dim(pad_h)?,
        dim(pad_w)?,
        dim(h_out)?,
        dim(w_out)?,
    ])
}

/// `RawTensor::gpu_matmul` (`src/ops/gpu_ops.rs:151-169`): c[m,n] = a[m,k] . b[k,n].
#[allow(clippy::many_single_char_names)]
pub fn gpu_matmul(a: &DeviceBuffer, b: &DeviceBuffer, m: usize, k: usize, n: usize) -> Option<DeviceBuffer> {
    let dt = same_dtype(a, b)?;
    let (mi, ki, ni) = (dim(m)?, dim(k)?, dim(n)?);
    // SAFETY: device pointers of live buffers; the library checks the sizes.
    alloc_out(count(&[m, n])?, dt, |out| unsafe { vh_matmul_alloc(dt, a.ptr, b.ptr, out, mi, ki, ni, STREAM) })
}

/// `RawTensor::gpu_matmul_backward_a` (`src/ops/gpu_ops.rs:408-428`):
/// grad_a[m,k] = grad[m,n] . b[k,n]^T.
#[allow(clippy::many_single_char_names)]
pub fn gpu_matmul_backward_a(grad: &DeviceBuffer, b: &DeviceBuffer, m: usize, k: usize, n: usize) -> Option<DeviceBuffer> {
    let dt = same_dtype(grad, b)?;
    let (mi, ki, ni) = (dim(m)?, dim(k)?, dim(n)?);
    // SAFETY: as gpu_matmul.
    alloc_out(count(&[m, k])?, dt, |out| unsafe {
        vh_matmul_backward_a_alloc(dt, grad.ptr, b.ptr, out, mi, ki, ni, STREAM)
    })
}

/// `RawTensor::gpu_matmul_backward_b` (`src/ops/gpu_ops.rs:430-450`):
/// grad_b[k,n] = a[m,k]^T . grad[m,n].
#[allow(clippy::many_single_char_names)]
pub fn gpu_matmul_backward_b(a: &DeviceBuffer, grad: &DeviceBuffer, m: usize, k: usize, n: usize) -> Option<DeviceBuffer> {
    let dt = same_dtype(a, grad)?;
    let (mi, ki, ni) = (dim(m)?, dim(k)?, dim(n)?);
    // SAFETY: as gpu_matmul.
    alloc_out(count(&[k, n])?, dt, |out| unsafe {
        vh_matmul_backward_b_alloc(dt, a.ptr, grad.ptr, out, mi, ki, ni, STREAM)
    })
}

/// `RawTensor::gpu_im2col` (`src/ops/gpu_ops.rs:515-544`): rows (b, p, q),
/// columns (c, r, s) of an already padded input.
#[allow(clippy::too_many_arguments)]
pub fn gpu_im2col(
    input: &DeviceBuffer,
    batch_size: usize,
    channels: usize,
    height: usize,
    width: usize,
    kernel_h: usize,
    kernel_w: usize,
    stride_h: usize,
    stride_w: usize,
    h_out: usize,
    w_out: usize,
) -> Option<DeviceBuffer> {
    let dt = input.dtype;
    let d = [
        dim(batch_size)?,
        dim(channels)?,
        dim(height)?,
        dim(width)?,
        dim(kernel_h)?,
        dim(kernel_w)?,
        dim(stride_h)?,
        dim(stride_w)?,
        dim(h_out)?,
        dim(w_out)?,
    ];
    let len = count(&[batch_size, h_out, w_out, channels, kernel_h, kernel_w])?;
    // SAFETY: device pointer of a live buffer; the library checks the sizes.
    alloc_out(len, dt, |out| unsafe {
        vh_im2col_alloc(dt, input.ptr, out, d[0], d[1], d[2], d[3], d[4], d[5], d[6], d[7], d[8], d[9], STREAM)
    })
}

/// `RawTensor::gpu_col2im` (`src/ops/gpu_ops.rs:546-572`): the scatter-add adjoint of im2col.
#[allow(clippy::too_many_arguments)]
pub fn gpu_col2im(
    col: &DeviceBuffer,
    batch_size: usize,
    channels: usize,
    height: usize,
    width: usize,
    kernel_h: usize,
    kernel_w: usize,
    stride_h: usize,
    stride_w: usize,
    h_out: usize,
    w_out: usize,
) -> Option<DeviceBuffer> {
    let dt = col.dtype;
    let d = [
        dim(batch_size)?,
        dim(channels)?,
        dim(height)?,
        dim(width)?,
        dim(kernel_h)?,
        dim(kernel_w)?,
        dim(stride_h)?,
        dim(stride_w)?,
        dim(h_out)?,
        dim(w_out)?,
    ];
    let len = count(&[batch_size, channels, height, width])?;
    // SAFETY: as gpu_im2col.
    alloc_out(len, dt, |out| unsafe {
        vh_col2im_alloc(dt, col.ptr, out, d[0], d[1], d[2], d[3], d[4], d[5], d[6], d[7], d[8], d[9], STREAM)
    })
}

/// Signature shared by the allocating convolution entry points.
type ConvAllocFn = unsafe extern "C" fn(
    c_int,
    *const c_void,
    *const c_void,
    *mut *mut c_void,
    i64,
    i64,
    i64,
    i64,
    i64,
    i64,
    i64,
    i64,
    i64,
    i64,
    i64,
    i64,
    i64,
    *mut c_void,
) -> c_int;

/// Calls one allocating convolution entry point with two operands and the 13
/// dimensions; the output has `len` elements.
fn conv_call(f: ConvAllocFn, t0: &DeviceBuffer, t1: &DeviceBuffer, d: [i64; 13], len: usize) -> Option<DeviceBuffer> {
    let dt = same_dtype(t0, t1)?;
    // SAFETY: device pointers of live buffers; the library checks the sizes.
    alloc_out(len, dt, |out| unsafe {
        f(dt, t0.ptr, t1.ptr, out, d[0], d[1], d[2], d[3], d[4], d[5], d[6], d[7], d[8], d[9], d[10], d[11], d[12], STREAM)
    })
}

/// `RawTensor::gpu_direct_conv` (`src/ops/gpu_ops.rs:574-620`): the Direct
/// forward (stride before pad, as the reference's `gpu_*` functions take them).
#[allow(clippy::too_many_arguments)]
pub fn gpu_direct_conv(
    input: &DeviceBuffer,
    weight: &DeviceBuffer,
    batch_size: usize,
    in_channels: usize,
    out_channels: usize,
    height: usize,
    width: usize,
    kernel_h: usize,
    kernel_w: usize,
    stride_h: usize,
    stride_w: usize,
    pad_h: usize,
    pad_w: usize,
    h_out: usize,
    w_out: usize,
) -> Option<DeviceBuffer> {
    let d = conv_dims(batch_size, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w, h_out, w_out)?;
    let len = count(&[batch_size, out_channels, h_out, w_out])?;
    conv_call(vh_direct_conv_alloc, input, weight, d, len)
}

/// `RawTensor::gpu_igemm` (`src/ops/gpu_ops.rs:622-668`): the implicit-GEMM forward.
#[allow(clippy::too_many_arguments)]
pub fn gpu_igemm(
    input: &DeviceBuffer,
    weight: &DeviceBuffer,
    batch_size: usize,
    in_channels: usize,
    out_channels: usize,
    height: usize,
    width: usize,
    kernel_h: usize,
    kernel_w: usize,
    stride_h: usize,
    stride_w: usize,
    pad_h: usize,
    pad_w: usize,
    h_out: usize,
    w_out: usize,
) -> Option<DeviceBuffer> {
    let d = conv_dims(batch_size, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w, h_out, w_out)?;
    let len = count(&[batch_size, out_channels, h_out, w_out])?;
    conv_call(vh_igemm_alloc, input, weight, d, len)
}

/// `RawTensor::gpu_conv_backward_input` (`src/ops/gpu_ops.rs:670-716`): the
/// Direct algorithm's input gradient.
#[allow(clippy::too_many_arguments)]
pub fn gpu_conv_backward_input(
    out_grad: &DeviceBuffer,
    weight: &DeviceBuffer,
    batch_size: usize,
    in_channels: usize,
    out_channels: usize,
    height: usize,
    width: usize,
    kernel_h: usize,
    kernel_w: usize,
    stride_h: usize,
    stride_w: usize,
    pad_h: usize,
    pad_w: usize,
    h_out: usize,
    w_out: usize,
) -> Option<DeviceBuffer> {
    let d = conv_dims(batch_size, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w, h_out, w_out)?;
    let len = count(&[batch_size, in_channels, height, width])?;
    conv_call(vh_conv_backward_input_alloc, out_grad, weight, d, len)
}

/// `RawTensor::gpu_conv_backward_weight` (`src/ops/gpu_ops.rs:718-764`): the
/// Direct algorithm's weight gradient, `(out_grad, input)` in that order.
#[allow(clippy::too_many_arguments)]
pub fn gpu_conv_backward_weight(
    out_grad: &DeviceBuffer,
    input: &DeviceBuffer,
    batch_size: usize,
    in_channels: usize,
    out_channels: usize,
    height: usize,
    width: usize,
    kernel_h: usize,
    kernel_w: usize,
    stride_h: usize,
    stride_w: usize,
    pad_h: usize,
    pad_w: usize,
    h_out: usize,
    w_out: usize,
) -> Option<DeviceBuffer> {
    let d = conv_dims(batch_size, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w, h_out, w_out)?;
    let len = count(&[out_channels, in_channels, kernel_h, kernel_w])?;
    conv_call(vh_conv_backward_weight_alloc, out_grad, input, d, len)
}

/// `RawTensor::gpu_igemm_backward_input` (`src/ops/gpu_ops.rs:766-812`).
#[allow(clippy::too_many_arguments)]
pub fn gpu_igemm_backward_input(
    out_grad: &DeviceBuffer,
    weight: &DeviceBuffer,
    batch_size: usize,
    in_channels: usize,
    out_channels: usize,
    height: usize,
    width: usize,
    kernel_h: usize,
    kernel_w: usize,
    stride_h: usize,
    stride_w: usize,
    pad_h: usize,
    pad_w: usize,
    h_out: usize,
    w_out: usize,
) -> Option<DeviceBuffer> {
    let d = conv_dims(batch_size, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w, h_out, w_out)?;
    let len = count(&[batch_size, in_channels, height, width])?;
    conv_call(vh_igemm_backward_input_alloc, out_grad, weight, d, len)
}

/// `RawTensor::gpu_igemm_backward_weight` (`src/ops/gpu_ops.rs:814-861`),
/// `(out_grad, input)` in that order.
#[allow(clippy::too_many_arguments)]
pub fn gpu_igemm_backward_weight(
    out_grad: &DeviceBuffer,
    input: &DeviceBuffer,
    batch_size: usize,
    in_channels: usize,
    out_channels: usize,
    height: usize,
    width: usize,
    kernel_h: usize,
    kernel_w: usize,
    stride_h: usize,
    stride_w: usize,
    pad_h: usize,
    pad_w: usize,
    h_out: usize,
    w_out: usize,
) -> Option<DeviceBuffer> {
    let d = conv_dims(batch_size, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w, h_out, w_out)?;
    let len = count(&[out_channels, in_channels, kernel_h, kernel_w])?;
    conv_call(vh_igemm_backward_weight_alloc, out_grad, input, d, len)
}

/// The unary ops this library implements, by the reference's op names.
fn unary_op(op: &str) -> Option<c_int> {
    match op {
        "relu" => Some(VH_UNARY_RELU),
        _ => None,
    }
}

/// `RawTensor::gpu_unary` (`src/ops/gpu_ops.rs:171-184`) for "relu"; other ops
/// return `None` (the CPU path).
pub fn gpu_unary(input: &DeviceBuffer, op: &str) -> Option<DeviceBuffer> {
    let code = unary_op(op)?;
    let dt = input.dtype;
    let n = dim(input.len)?;
    let mut out = DeviceBuffer::new(input.len, dt)?;
    // SAFETY: both buffers hold `input.len` elements of `dt`.
    check(unsafe { vh_unary(dt, code, input.ptr, out.as_mut_ptr(), n, STREAM) }).ok()?;
    Some(out)
}

/// `RawTensor::gpu_unary_backward` (`src/ops/gpu_ops.rs:186-200`) for "relu".
pub fn gpu_unary_backward(out_grad: &DeviceBuffer, x: &DeviceBuffer, op: &str) -> Option<DeviceBuffer> {
    let code = unary_op(op)?;
    let dt = same_dtype(out_grad, x)?;
    if out_grad.len != x.len {
        return None;
    }
    let n = dim(x.len)?;
    let mut out = DeviceBuffer::new(x.len, dt)?;
    // SAFETY: all three buffers hold `x.len` elements of `dt`.
    check(unsafe { vh_unary_backward(dt, code, out_grad.ptr, x.ptr, out.as_mut_ptr(), n, STREAM) }).ok()?;
    Some(out)
}

/// `RawTensor::gpu_sum_reduce` (`src/ops/gpu_ops.rs:118-121`): the sum of every element.
pub fn gpu_sum_reduce(data: &DeviceBuffer) -> Option<f32> {
    let n = dim(data.len)?;
    let mut res = DeviceBuffer::new(1, VH_F32)?;
    // SAFETY: `res` holds one f32; `data` holds `data.len` elements of its dtype.
    check(unsafe { vh_sum_reduce(data.dtype, data.ptr, n, res.as_mut_ptr() as *mut f32, STREAM) }).ok()?;
    res.to_f32_vec()?.first().copied()
}

/// `RawTensor::gpu_sum_backward` (`src/ops/gpu_ops.rs:452-463`): `input_size`
/// f32 elements equal to `grad` (with grad = 1, the autograd seed).
pub fn gpu_sum_backward(grad: f32, input_size: usize) -> Option<DeviceBuffer> {
    let n = dim(input_size)?;
    let mut out = DeviceBuffer::new(input_size, VH_F32)?;
    // SAFETY: `out` holds `input_size` f32 elements.
    check(unsafe { vh_sum_backward(VH_F32, grad, out.as_mut_ptr(), n, STREAM) }).ok()?;
    Some(out)
}
