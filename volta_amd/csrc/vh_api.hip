// vh_api.hip -- extern "C" entry points of libvolta_hip.so (declared in
// include/volta_hip.h), the device-memory runtime behind them, and the
// layer-level host logic (algorithm selection, Conv2d / ConvTranspose2d /
// Linear forward and backward composition) that Volta keeps in
// src/nn/layers/{conv,conv_transpose,linear}.rs.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "vh_kernels.hpp"

namespace vh {

static thread_local char g_err[512] = "";

int set_error(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return status;
}

// Specialised kernels (halo conv, ...) are used where their envelope allows
// unless the policy says otherwise (vh_set_kernel_policy; the environment
// variable VOLTA_HIP_GENERIC=1 sets the initial policy to generic).
static bool g_fast_paths = [] {
  const char* e = getenv("VOLTA_HIP_GENERIC");
  return !(e && e[0] == '1');
}();

// ------------------------------------------------------------------ device init
static std::once_flag g_init_once;
static int g_init_status = VH_ERR_NO_DEVICE;
static int scratch_ptr(void** out);

static int ensure_init() {
  std::call_once(g_init_once, [] {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
      g_init_status = VH_ERR_NO_DEVICE;
      return;
    }
    g_init_status = VH_OK;
  });
  if (g_init_status == VH_OK) {
    // the static scratch of the current device (other devices: on their first no-alloc call)
    static std::once_flag scratch_once;
    std::call_once(scratch_once, [] {
      void* p;
      (void)scratch_ptr(&p);
    });
  }
  if (g_init_status != VH_OK) return set_error(g_init_status, "no HIP device available");
  return VH_OK;
}

// ------------------------------------------------------------------ buffer pool
// Freed buffers up to 64 MiB are kept in size buckets (at most 8 per bucket, 64
// in total) and handed out again, like the reference's pool (src/gpu/pool.rs:28-35).
struct Pool {
  std::mutex mu;
  std::multimap<size_t, void*> free_list;
  std::unordered_map<void*, size_t> live;
  size_t cached = 0;
};
static Pool g_pool;
static constexpr size_t kPoolMaxBytes = 64u << 20;
static constexpr size_t kPoolMaxCount = 64;

static size_t round_bytes(size_t b) { return (b + 255) & ~size_t(255); }

// ------------------------------------------------------------------ per-stream workspace
// One grow-only device buffer per HIP stream; stream order makes its reuse by
// consecutive calls on that stream safe.  A HIP graph captured on the stream
// records the buffer's address, so its replays use the capture stream's
// buffer wherever they run.  A buffer that a later call outgrows is therefore
// freed (after the stream's queued work, which may still use it) only when no
// call was captured while it was current; a buffer that a capture referenced is
// retired instead and freed only by vh_release_cache(), which is why a release
// invalidates every graph captured from library calls.  While the stream is
// being captured the workspace never grows (that would allocate, and
// synchronise nothing, in the middle of a capture): the call fails with
// VH_ERR_CAPTURE and the caller runs it once eagerly before capturing.
struct Ws {
  void* ptr = nullptr;
  size_t bytes = 0;
  bool captured = false;  // a call captured into a graph used this buffer
};
static std::mutex g_ws_mu;
static std::unordered_map<hipStream_t, Ws> g_ws;
static std::vector<void*> g_ws_retired;

// Set by the allocation-free entry point for the duration of one call on the
// calling thread: ws_get then serves every request from this fixed buffer.
static thread_local void* t_ws_fixed = nullptr;
static thread_local size_t t_ws_fixed_bytes = 0;

// Growth rule of ws_get: the new size to allocate, or 0 when `have` suffices.
static size_t ws_grow_to(size_t have, size_t need) {
  if (need <= have) return 0;
  return round_bytes(std::max(need, have * 5 / 4));
}

// Returns a device buffer of >= bytes private to `st`.
static int ws_get(hipStream_t st, size_t bytes, void** out) {
  *out = nullptr;
  if (bytes == 0) return VH_OK;
  if (t_ws_fixed) {
    if (bytes > t_ws_fixed_bytes)
      return set_error(VH_ERR_UNSUPPORTED, "call needs %zu bytes of scratch; the static scratch holds %zu", bytes,
                       t_ws_fixed_bytes);
    *out = t_ws_fixed;
    return VH_OK;
  }
  std::lock_guard<std::mutex> lk(g_ws_mu);
  Ws& w = g_ws[st];
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  VH_HIP_CHECK(hipStreamIsCapturing(st, &cs));
  const bool capturing = cs != hipStreamCaptureStatusNone;
  const size_t nb = ws_grow_to(w.bytes, bytes);
  if (nb) {
    if (capturing)
      return set_error(VH_ERR_CAPTURE,
                       "workspace of this stream (%zu bytes) must grow to %zu while the stream is captured: "
                       "run the call once eagerly on the stream before capturing",
                       w.bytes, bytes);
    if (w.ptr) {
      void* old = w.ptr;
      const bool keep = w.captured;
      w.ptr = nullptr;
      w.bytes = 0;
      w.captured = false;
      if (keep) {
        g_ws_retired.push_back(old);  // a graph holds its address: freed by vh_release_cache only
      } else {
        // only this stream's queued calls can still use it
        const hipError_t e = hipStreamSynchronize(st);
        if (e != hipSuccess) {
          g_ws_retired.push_back(old);
          return set_error(VH_ERR_LAUNCH, "hipStreamSynchronize before a workspace grows failed: %s",
                           hipGetErrorString(e));
        }
        VH_HIP_CHECK(hipFree(old));
      }
    }
    void* p = nullptr;
    if (hipMalloc(&p, nb) != hipSuccess) {
      (void)hipGetLastError();
      return set_error(VH_ERR_OOM, "workspace allocation of %zu bytes failed", nb);
    }
    w.ptr = p;
    w.bytes = nb;
    w.captured = false;
  }
  if (capturing) w.captured = true;
  *out = w.ptr;
  return VH_OK;
}

// Carves aligned sub-buffers out of one workspace request.
struct Carve {
  size_t off = 0;
  size_t take(size_t bytes) {
    size_t o = off;
    off += round_bytes(bytes);
    return o;
  }
};

static inline char* at(void* base, size_t off) { return static_cast<char*>(base) + off; }

// ------------------------------------------------------------------ static scratch
// Device memory of the allocation-free entry point vh_conv2d_backward_noalloc:
// a fixed array in the code object's zero-initialised data, one copy per GPU.
// In host code `scratch` names a host-side stand-in, not device memory: its
// device address comes from hipGetSymbolAddress, once per device with that
// device current, and only that address is ever passed to kernels.
static constexpr size_t kScratchBytes = VH_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
static constexpr int kMaxDevices = 64;
static std::once_flag g_scratch_once[kMaxDevices];
static void* g_scratch_ptr[kMaxDevices];
static hipError_t g_scratch_err[kMaxDevices];

// Device address of the current device's scratch (set-up on first use per device).
static int scratch_ptr(void** out) {
  *out = nullptr;
  int dev = 0;
  VH_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return set_error(VH_ERR_UNSUPPORTED, "device %d beyond the scratch table", dev);
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? p : nullptr;
  });
  if (g_scratch_err[dev] != hipSuccess || !g_scratch_ptr[dev])
    return set_error(VH_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                     hipGetErrorString(g_scratch_err[dev]));
  *out = g_scratch_ptr[dev];
  return VH_OK;
}

// Routes every workspace request of the calling thread to a fixed buffer for the
// lifetime of the guard (ws_get never allocates while it is active).
struct FixedWs {
  FixedWs(void* p, size_t bytes) {
    t_ws_fixed = p;
    t_ws_fixed_bytes = bytes;
  }
  ~FixedWs() {
    t_ws_fixed = nullptr;
    t_ws_fixed_bytes = 0;
  }
};

// ------------------------------------------------------------------ validation
static constexpr long kMaxElems = (1L << 31) - 1;

static int elem_size(int dtype) { return dtype == VH_BF16 ? 2 : 4; }

static int check_dtype(int dtype) {
  if (dtype != VH_F32 && dtype != VH_BF16) return set_error(VH_ERR_BAD_ARG, "unknown dtype %d", dtype);
  return VH_OK;
}

static int check_sizes(std::initializer_list<long> sizes) {
  for (long s : sizes) {
    if (s < 0) return set_error(VH_ERR_BAD_SHAPE, "negative tensor size");
    if (s > kMaxElems) return set_error(VH_ERR_UNSUPPORTED, "tensor of %ld elements exceeds 2^31-1", s);
  }
  return VH_OK;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

struct ConvDims {
  long B, C, O, H, W, KH, KW, SH, SW, PH, PW, HO, WO;
};

static int conv_out_dim(long in, long k, long s, long p, long* out) {
  if (k <= 0 || s <= 0 || p < 0) return set_error(VH_ERR_BAD_SHAPE, "bad kernel/stride/padding");
  if (in + 2 * p < k) return set_error(VH_ERR_BAD_SHAPE, "input (%ld, pad %ld) smaller than kernel %ld", in, p, k);
  *out = (in + 2 * p - k) / s + 1;
  return VH_OK;
}

static int check_conv(const ConvDims& d, bool check_out) {
  if (d.B < 0 || d.C <= 0 || d.O <= 0 || d.H <= 0 || d.W <= 0)
    return set_error(VH_ERR_BAD_SHAPE, "bad conv dimensions");
  long ho, wo;
  int st;
  if ((st = conv_out_dim(d.H, d.KH, d.SH, d.PH, &ho))) return st;
  if ((st = conv_out_dim(d.W, d.KW, d.SW, d.PW, &wo))) return st;
  if (check_out && (ho != d.HO || wo != d.WO))
    return set_error(VH_ERR_BAD_SHAPE, "h_out/w_out (%ld,%ld) do not match geometry (%ld,%ld)", d.HO, d.WO, ho, wo);
  return check_sizes({d.B * d.C * d.H * d.W, d.B * d.O * ho * wo, d.O * d.C * d.KH * d.KW});
}

static ConvGeom geom_of(const ConvDims& d) {
  return make_geom((int)d.B, (int)d.C, (int)d.H, (int)d.W, (int)d.O, (int)d.KH, (int)d.KW, (int)d.HO, (int)d.WO,
                   (int)d.SH, (int)d.SW, (int)d.PH, (int)d.PW);
}

#define VH_TRY(expr)          \
  do {                        \
    int _s = (expr);          \
    if (_s != VH_OK) return _s; \
  } while (0)

#define VH_DISPATCH(dtype, FN, ...) \
  ((dtype) == VH_BF16 ? FN<bf16>(__VA_ARGS__) : FN<float>(__VA_ARGS__))

// ------------------------------------------------------------------ conv passes
// 1x1 kernel, no padding, equal strides >= 2 (the ResNet projection shortcut).
static bool is_strided_pointwise(const ConvDims& d) {
  return d.KH == 1 && d.KW == 1 && d.PH == 0 && d.PW == 0 && d.SH == d.SW && d.SH >= 2;
}

// Forward pass as implicit GEMM: rows = output channels (A = weight in
// [O][kh][kw][C] order), columns = output positions (B = im2col gather of x).
// ReLU applied in place after a pass whose kernel has no fused epilogue for it.
static int relu_after(int dt, void* y, long n, hipStream_t st) {
  return VH_DISPATCH(dt, run_relu, y, nullptr, y, n, st);
}
// grad = mask > 0 ? grad : 0 in place (the ReLU backward of the layer below).
static int mask_after(int dt, const void* mask, void* grad, long n, hipStream_t st) {
  return VH_DISPATCH(dt, run_relu, mask, grad, grad, n, st);
}

static bool is_3x3_s1_p1(const ConvDims& d) {
  return d.KH == 3 && d.KW == 3 && d.SH == 1 && d.SW == 1 && d.PH == 1 && d.PW == 1;
}

// act: 1 = ReLU on the output (fused into the epilogue where the kernel has it).
static int igemm_fwd(int dt, const void* x, const void* w, const void* bias, void* y, const ConvDims& d,
                     hipStream_t st, int act = 0) {
  if (dt == VH_BF16 && is_strided_pointwise(d) && g_fast_paths) {
    int r = pw_conv_bf16_fwd(x, w, bias, y, (int)d.B, (int)d.C, (int)d.H, (int)d.W, (int)d.O, (int)d.SH, st);
    if (r != VH_ERR_UNSUPPORTED) return r == VH_OK && act ? relu_after(dt, y, d.B * d.O * d.HO * d.WO, st) : r;
  }
  ConvGeom g = geom_of(d);
  const long RS = d.KH * d.KW;
  if (dt == VH_F32 && g_fast_paths) {
    // 4x4 stride 2 from a few channels (the up-sampling layer's input gradient)
    int r = cell_fwd_f32(x, w, bias, y, g, act, st);
    if (r != VH_ERR_UNSUPPORTED) return r;
    if (is_3x3_s1_p1(d)) {  // narrow images: the fp32 halo kernel
      r = halo_conv3x3_f32(x, w, 0, bias, nullptr, y, (int)d.B, (int)d.C, (int)d.H, (int)d.W, (int)d.O, act, st);
      if (r != VH_ERR_UNSUPPORTED) return r;
    }
  }
  // weight staging: the generic layout, or the halo kernel's channel-grouped one (padded to 16 channels)
  const size_t wbytes = std::max((size_t)d.O * d.C * RS * elem_size(dt),
                                 halo_conv_bf16_ws((int)d.C, (int)d.O, (int)d.KH, (int)d.KW));
  IgemmPlan p{};
  p.dtype = dt;
  p.akind = KD_DENSE_K;
  p.bkind = KD_CONV_FWD_X;
  p.okind = OK_NCHW;
  p.args.M = (int)d.O;
  p.args.N = (int)(d.B * d.HO * d.WO);
  p.args.K = (int)(RS * d.C);
  p.args.g = g;
  p.args.hwo = (int)(d.HO * d.WO);
  p.args.f_hwo = FastDiv((uint32_t)std::max<long>(1, d.HO * d.WO));
  p.args.bias = bias;
  p.args.bias_mode = bias ? 1 : 0;
  p.args.d = y;
  p.splits = pick_splits(p.args.M, p.args.N, p.args.K, dt);
  size_t ws_gemm = igemm_prepare(p);
  Carve cv;
  size_t o_w = cv.take(wbytes), o_g = cv.take(ws_gemm);
  void* ws;
  VH_TRY(ws_get(st, cv.off, &ws));
  void* wt = at(ws, o_w);
  if (dt == VH_BF16 && d.SH == 1 && d.SW == 1 && g_fast_paths && d.C <= 4 && act <= 1) {
    // few input channels: K packed as (c, r, s) instead of 16-channel groups
    int r = smallc_conv_bf16(x, w, bias, y, (int)d.B, (int)d.C, (int)d.H, (int)d.W, (int)d.O, (int)d.KH, (int)d.KW,
                             (int)d.PH, (int)d.PW, act, st);
    if (r != VH_ERR_UNSUPPORTED) return r;
  }
  if (dt == VH_BF16 && d.SH == 1 && d.SW == 1 && g_fast_paths) {
    int r = halo_conv_bf16(x, w, 0, wt, bias, y, (int)d.B, (int)d.C, (int)d.H, (int)d.W, (int)d.O, (int)d.KH,
                           (int)d.KW, (int)d.PH, (int)d.PW, st, act);
    if (r != VH_ERR_UNSUPPORTED) return r;
  }
  VH_TRY(VH_DISPATCH(dt, run_relayout, w, wt, (int)d.O, (int)d.C, (int)RS, 0, st));
  const int vec = dt == VH_BF16 ? 8 : 4;
  p.args.a = Operand{wt, (int)(RS * d.C), (int)d.O, ((RS * d.C) % vec) == 0};
  p.args.b = Operand{x, 0, p.args.N, 0};
  p.args.act = act;
  return run_igemm(p, (float*)at(ws, o_g), st);
}

// Input gradient of a strided convolution (and ConvTranspose2d's forward), one
// stride phase at a time: input positions (a + sh*i, b + sw*j) receive only the
// taps kh = (a + ph) mod sh + sh*t (and likewise kw), so each phase is a stride-1
// implicit GEMM over its Rc x Sc taps with padding (a + ph - kh0) / sh, storing
// into the phase's positions (OK_NCHW_SUB) -- 1/(sh*sw) of the MFMA work of the
// dense tap loop, whose other taps multiply zeros. A phase without taps stores
// zeros (plus the bias). The phases run in order on one stream, sharing one
// workspace.
struct DgradPhase {
  int a, b, Hc, Wc, kh0, kw0, Rc, Sc, offa, offb;
};

// need != nullptr: sizing mode -- stores the workspace bytes the call would
// request and returns without launching anything (same for the passes below).
static int dgrad_phases(int dt, const void* dy, const void* w, const void* bias, void* dx, const ConvDims& d,
                        hipStream_t st, const void* mask = nullptr, size_t* need = nullptr) {
  const int SH = (int)d.SH, SW = (int)d.SW;
  std::vector<DgradPhase> ph;
  PhaseTable tab{};
  size_t wtot = 0, gmax = 0;
  for (int a = 0; a < SH && a < d.H; ++a)
    for (int b = 0; b < SW && b < d.W; ++b) {
      DgradPhase f;
      f.a = a;
      f.b = b;
      f.Hc = (int)((d.H - a + SH - 1) / SH);
      f.Wc = (int)((d.W - b + SW - 1) / SW);
      f.kh0 = (int)((a + d.PH) % SH);
      f.kw0 = (int)((b + d.PW) % SW);
      f.Rc = f.kh0 < d.KH ? (int)((d.KH - f.kh0 + SH - 1) / SH) : 0;
      f.Sc = f.kw0 < d.KW ? (int)((d.KW - f.kw0 + SW - 1) / SW) : 0;
      f.offa = (int)((a + d.PH - f.kh0) / SH);
      f.offb = (int)((b + d.PW - f.kw0) / SW);
      const long K = (long)f.Rc * f.Sc * d.O;
      if (tab.n == 16) return VH_ERR_UNSUPPORTED;
      tab.kh0[tab.n] = f.kh0;
      tab.kw0[tab.n] = f.kw0;
      tab.rc[tab.n] = f.Rc;
      tab.sc[tab.n] = f.Sc;
      tab.off[tab.n] = (long)(wtot / elem_size(dt));
      ++tab.n;
      wtot += round_bytes((size_t)K * d.C * elem_size(dt));
      IgemmPlan p{};
      p.dtype = dt;
      p.args.M = (int)d.C;
      p.args.N = (int)(d.B * f.Hc * f.Wc);
      p.args.K = (int)K;
      p.splits = pick_splits(p.args.M, p.args.N, p.args.K, dt);
      gmax = std::max(gmax, igemm_prepare(p));
      ph.push_back(f);
    }
  Carve cv;
  const size_t o_w = cv.take(std::max<size_t>(wtot, 16)), o_g = cv.take(gmax);
  if (need) {
    *need = cv.off;
    return VH_OK;
  }
  void* ws;
  VH_TRY(ws_get(st, cv.off, &ws));
  VH_TRY(VH_DISPATCH(dt, run_relayout_phase, w, at(ws, o_w), (int)d.O, (int)d.C, (int)d.KH, (int)d.KW, SH, SW, tab,
                     st));
  const int vec = dt == VH_BF16 ? 8 : 4;
  // Phases of one shape (every phase has taps, equal extents): one launch with
  // the phase in blockIdx.y, when the phases' tiles together fill the chip
  // without split K.
  bool uniform = ph.size() >= 2 && ph.size() <= 4;
  for (size_t pi = 0; uniform && pi < ph.size(); ++pi)
    uniform = ph[pi].Rc > 0 && ph[pi].Sc > 0 && ph[pi].Rc == ph[0].Rc && ph[pi].Sc == ph[0].Sc &&
              ph[pi].Hc == ph[0].Hc && ph[pi].Wc == ph[0].Wc;
  for (size_t pi = 0; pi < ph.size(); ++pi) {
    const DgradPhase& f = ph[pi];
    const int K = f.Rc * f.Sc * (int)d.O;
    const void* wp = at(ws, o_w + (size_t)tab.off[pi] * elem_size(dt));
    IgemmPlan p{};
    p.dtype = dt;
    p.akind = KD_DENSE_K;
    p.bkind = KD_CONV_DGRAD_DY;
    p.okind = OK_NCHW_SUB;
    p.args.M = (int)d.C;
    p.args.N = (int)(d.B * f.Hc * f.Wc);
    p.args.K = K;
    p.args.g = make_geom((int)d.B, (int)d.C, f.Hc, f.Wc, (int)d.O, std::max(1, f.Rc), std::max(1, f.Sc), (int)d.HO,
                         (int)d.WO, 1, 1, f.offa, f.offb);
    p.args.hwo = f.Hc * f.Wc;
    p.args.f_hwo = FastDiv((uint32_t)(f.Hc * f.Wc));
    p.args.f_wsub = FastDiv((uint32_t)f.Wc);
    p.args.sub_sh = SH;
    p.args.sub_sw = SW;
    p.args.sub_a = f.a;
    p.args.sub_b = f.b;
    p.args.sub_H = (int)d.H;
    p.args.sub_W = (int)d.W;
    p.args.d = dx;
    p.args.bias = bias;
    p.args.bias_mode = bias ? 1 : 0;
    p.args.act = mask ? 2 : 0;
    p.args.mask = mask;
    p.splits = pick_splits(p.args.M, p.args.N, p.args.K, dt);
    p.args.a = Operand{wp, std::max(K, 1), (int)d.C, (K % vec) == 0};
    p.args.b = Operand{dy, 0, p.args.N, 0};
    if (uniform && pi == 0 && pick_splits(p.args.M, p.args.N * (int)ph.size(), p.args.K, dt) == 1) {
      p.splits = 1;
      p.args.nphase = (int)ph.size();
      for (size_t q = 0; q < ph.size(); ++q)
        p.args.ph[q] = PhaseArg{at(ws, o_w + (size_t)tab.off[q] * elem_size(dt)), ph[q].offa, ph[q].offb, ph[q].a,
                                ph[q].b};
      igemm_prepare(p);
      return run_igemm(p, (float*)at(ws, o_g), st);
    }
    igemm_prepare(p);
    VH_TRY(run_igemm(p, (float*)at(ws, o_g), st));
  }
  return VH_OK;
}

// Input gradient as implicit GEMM: rows = input channels (A = weight in
// [C][kh][kw][O] order), columns = input positions (B = gather of dY).
// mask: the layer input, when it came from a ReLU: dx is zeroed where it is not
// positive (the ReLU backward of the layer below, fused where the kernel has it).
static int igemm_dgrad(int dt, const void* dy, const void* w, void* dx, const ConvDims& d, hipStream_t st,
                       const void* mask = nullptr, size_t* need = nullptr) {
  ConvGeom g = geom_of(d);
  const long RS = d.KH * d.KW;
  const size_t wbytes = std::max((size_t)d.O * d.C * RS * elem_size(dt),
                                 halo_conv_bf16_ws((int)d.O, (int)d.C, (int)d.KH, (int)d.KW));
  IgemmPlan p{};
  p.dtype = dt;
  p.akind = KD_DENSE_K;
  p.bkind = KD_CONV_DGRAD_DY;
  p.okind = OK_NCHW;
  p.args.M = (int)d.C;
  p.args.N = (int)(d.B * d.H * d.W);
  p.args.K = (int)(RS * d.O);
  p.args.g = g;
  p.args.hwo = (int)(d.H * d.W);
  p.args.f_hwo = FastDiv((uint32_t)(d.H * d.W));
  p.args.d = dx;
  p.splits = pick_splits(p.args.M, p.args.N, p.args.K, dt);
  size_t ws_gemm = igemm_prepare(p);
  Carve cv;
  size_t o_w = cv.take(wbytes), o_g = cv.take(ws_gemm);
  const bool halo_f32 = dt == VH_F32 && g_fast_paths && is_3x3_s1_p1(d) &&
                        halo_conv3x3_f32_ok(dy, w, (int)d.B, (int)d.O, (int)d.H, (int)d.W, (int)d.C);
  if (need) {
    // at most 4 input channels: the one-lane-per-position kernel; fp32 3x3 of
    // narrow images: the halo kernel -- neither takes workspace
    if (g_fast_paths && (dgrad_smallc_ok(g) || halo_f32)) {
      *need = 0;
      return VH_OK;
    }
    // the larger of this pass's request and the stride-phase path's
    size_t n = cv.off, np = 0;
    if ((d.SH > 1 || d.SW > 1) && g_fast_paths && dgrad_phases(dt, dy, w, nullptr, dx, d, st, mask, &np) == VH_OK)
      n = std::max(n, np);
    *need = n;
    return VH_OK;
  }
  // at most 4 input channels: one lane per input position, no workspace
  if (g_fast_paths && dgrad_smallc_ok(g)) return VH_DISPATCH(dt, run_dgrad_smallc, dy, w, nullptr, mask, dx, g, st);
  if (halo_f32)  // dX = conv(dY, W rotated, O and C swapped), the ReLU mask in the epilogue
    return halo_conv3x3_f32(dy, w, 1, nullptr, mask, dx, (int)d.B, (int)d.O, (int)d.H, (int)d.W, (int)d.C, 0, st);
  void* ws;
  VH_TRY(ws_get(st, cv.off, &ws));
  void* wd = at(ws, o_w);
  if (dt == VH_BF16 && d.SH == 1 && d.SW == 1 && d.PH <= d.KH - 1 && d.PW <= d.KW - 1 && g_fast_paths) {
    // stride 1: dX = conv(dY, W rotated 180 degrees with O and C swapped), pad K-1-p
    int r = halo_conv_bf16(dy, w, 1, wd, nullptr, dx, (int)d.B, (int)d.O, (int)d.HO, (int)d.WO, (int)d.C,
                           (int)d.KH, (int)d.KW, (int)(d.KH - 1 - d.PH), (int)(d.KW - 1 - d.PW), st,
                           mask ? 2 : 0, mask);
    if (r != VH_ERR_UNSUPPORTED) return r;
  }
  if (dt == VH_BF16 && is_strided_pointwise(d) && g_fast_paths && ((uintptr_t)dx & 3) == 0) {
    int r = pw_conv_bf16_dgrad(dy, w, dx, (int)d.B, (int)d.C, (int)d.H, (int)d.W, (int)d.O, (int)d.SH, st);
    if (r != VH_ERR_UNSUPPORTED) return r == VH_OK && mask ? mask_after(dt, mask, dx, d.B * d.C * d.H * d.W, st) : r;
  }
  if ((d.SH > 1 || d.SW > 1) && g_fast_paths) {
    int r = dgrad_phases(dt, dy, w, nullptr, dx, d, st, mask);  // unsupported only beyond 16 phases
    if (r != VH_ERR_UNSUPPORTED) return r;
  }
  VH_TRY(VH_DISPATCH(dt, run_relayout, w, wd, (int)d.O, (int)d.C, (int)RS, 1, st, 0));
  const int vec = dt == VH_BF16 ? 8 : 4;
  p.args.a = Operand{wd, (int)(RS * d.O), (int)d.C, ((RS * d.O) % vec) == 0};
  p.args.b = Operand{dy, 0, p.args.N, 0};
  p.args.act = mask ? 2 : 0;
  p.args.mask = mask;
  return run_igemm(p, (float*)at(ws, o_g), st);
}

// Weight gradient.  bf16 stride-1 layers use the row-streaming kernel
// (vh_wgrad.hip), which can also produce the bias gradient from the same pass
// (*db_done = true then); everything else runs the generic implicit GEMM with
// split-K over output positions: rows = O (A = dY), columns = (kh, kw, c)
// (B = gather of x), stored OIHW.
static int igemm_wgrad(int dt, const void* dy, const void* x, void* dw, void* db, bool* db_done,
                       const ConvDims& d, hipStream_t st, size_t* need = nullptr) {
  if (db_done) *db_done = false;
  size_t most = 0;  // sizing mode: the largest request of the paths that run
  if (dt == VH_BF16 && d.SH == 1 && d.SW == 1 && g_fast_paths) {
    size_t nb = wgrad_rows_ws((int)d.B, (int)d.C, (int)d.H, (int)d.W, (int)d.O, (int)d.KH, (int)d.KW,
                              (int)d.PH, (int)d.PW, db != nullptr);
    if (nb && need) {  // the row kernel runs whenever it plans a workspace
      *need = nb;
      return VH_OK;
    }
    if (nb) {
      void* ws;
      VH_TRY(ws_get(st, nb, &ws));
      int r = wgrad_rows_bf16(dy, x, dw, db, (int)d.B, (int)d.C, (int)d.H, (int)d.W, (int)d.O, (int)d.KH,
                              (int)d.KW, (int)d.PH, (int)d.PW, (float*)ws, nb, st);
      if (r != VH_ERR_UNSUPPORTED) {
        if (r == VH_OK && db_done) *db_done = db != nullptr;
        return r;
      }
    }
  }
  if (dt == VH_BF16 && is_strided_pointwise(d) && g_fast_paths) {
    size_t nb = pw_conv_bf16_wgrad_ws((int)d.B, (int)d.C, (int)d.H, (int)d.W, (int)d.O, (int)d.SH);
    if (nb && need && aligned16(x) && aligned16(dy)) {  // the pointwise kernel runs
      *need = nb;
      return VH_OK;
    }
    most = std::max(most, nb);  // requested, then unsupported for unaligned operands
    if (nb && !need) {
      void* ws;
      VH_TRY(ws_get(st, nb, &ws));
      int r = pw_conv_bf16_wgrad(dy, x, dw, (int)d.B, (int)d.C, (int)d.H, (int)d.W, (int)d.O, (int)d.SH,
                                 (float*)ws, nb, st);
      if (r != VH_ERR_UNSUPPORTED) return r;
    }
  }
  if (dt == VH_F32 && g_fast_paths && is_3x3_s1_p1(d)) {
    // fp32 3x3 of narrow images: the halo weight gradient (bias gradient included)
    const size_t nb = halo_wgrad3x3_f32_ws(dy, x, (int)d.B, (int)d.C, (int)d.H, (int)d.W, (int)d.O);
    if (nb && need) {
      *need = nb;
      return VH_OK;
    }
    if (nb) {
      void* ws;
      VH_TRY(ws_get(st, nb, &ws));
      int r = halo_wgrad3x3_f32(dy, x, dw, db, (int)d.B, (int)d.C, (int)d.H, (int)d.W, (int)d.O, (float*)ws, nb, st);
      if (r != VH_ERR_UNSUPPORTED) {
        if (r == VH_OK && db_done) *db_done = db != nullptr;
        return r;
      }
    }
  }
  ConvGeom g = geom_of(d);
  const long RS = d.KH * d.KW;
  IgemmPlan p{};
  p.dtype = dt;
  p.akind = KD_CONV_WGRAD_DY;
  p.bkind = KD_CONV_WGRAD_X;
  p.okind = OK_WGRAD_OIHW;
  p.args.M = (int)d.O;
  p.args.N = (int)(RS * d.C);
  p.args.K = (int)(d.B * d.HO * d.WO);
  p.args.g = g;
  p.args.wg_c = (int)d.C;
  p.args.wg_rs = (int)RS;
  p.args.f_cw = FastDiv((uint32_t)d.C);
  p.args.d = dw;
  p.args.a = Operand{dy, 0, (int)d.O, aligned16(dy)};
  p.args.b = Operand{x, 0, p.args.N, 0};
  if (db && p.args.N % 64 != 0) {
    // the bias gradient (row sums of dY) as one more column -- a B row of ones --
    // where it falls into the padding of the last column tile (no extra tile)
    p.args.N += 1;
    p.args.b = Operand{x, 1, p.args.N, 0};
    p.args.dbias = db;
  }
  p.wide = 1;
  p.splits = pick_splits(p.args.M, p.args.N, p.args.K, dt, p.wide);
  size_t ws_gemm = igemm_prepare(p);
  if (need) {
    *need = std::max(most, ws_gemm);
    return VH_OK;
  }
  void* ws;
  VH_TRY(ws_get(st, ws_gemm, &ws));
  const int r = run_igemm(p, (float*)ws, st);
  if (r == VH_OK && p.args.dbias && db_done) *db_done = true;
  return r;
}

static int bias_grad_nchw(int dt, const void* dy, void* db, long B, long C, long HW, hipStream_t st,
                          size_t* need = nullptr) {
  int ns;
  size_t bytes = channel_sum_ws((int)B, (int)C, (int)HW, &ns);
  if (need) {
    *need = bytes;
    return VH_OK;
  }
  void* ws;
  VH_TRY(ws_get(st, bytes, &ws));
  return VH_DISPATCH(dt, run_channel_sum, dy, (int)B, (int)C, (int)HW, db, (float*)ws, ns, st);
}

// Im2col forward (conv.rs:1858-1907): pad -> im2col -> W[O][CKK] . col^T -> NCHW.
static int im2col_fwd(int dt, const void* x, const void* w, const void* bias, void* y, const ConvDims& d,
                      hipStream_t st) {
  const long HP = d.H + 2 * d.PH, WP = d.W + 2 * d.PW, CKK = d.C * d.KH * d.KW;
  const long M = d.B * d.HO * d.WO;
  VH_TRY(check_sizes({M * CKK, d.B * d.C * HP * WP}));
  const int es = elem_size(dt);
  IgemmPlan p{};
  p.dtype = dt;
  p.akind = KD_DENSE_K;
  p.bkind = KD_DENSE_K;
  p.okind = OK_NCHW;
  p.args.M = (int)d.O;
  p.args.N = (int)M;
  p.args.K = (int)CKK;
  p.args.hwo = (int)(d.HO * d.WO);
  p.args.f_hwo = FastDiv((uint32_t)(d.HO * d.WO));
  p.args.bias = bias;
  p.args.bias_mode = bias ? 1 : 0;
  p.args.d = y;
  p.splits = pick_splits(p.args.M, p.args.N, p.args.K, dt);
  size_t ws_gemm = igemm_prepare(p);
  const bool padded = d.PH || d.PW;
  Carve cv;
  size_t o_xp = padded ? cv.take((size_t)d.B * d.C * HP * WP * es) : 0;
  size_t o_col = cv.take((size_t)M * CKK * es);
  size_t o_g = cv.take(ws_gemm);
  void* ws;
  VH_TRY(ws_get(st, cv.off, &ws));
  const void* xin = x;
  if (padded) {
    VH_TRY(VH_DISPATCH(dt, run_pad, x, at(ws, o_xp), (int)d.B, (int)d.C, (int)d.H, (int)d.W, (int)d.PH,
                       (int)d.PW, st));
    xin = at(ws, o_xp);
  }
  void* col = at(ws, o_col);
  VH_TRY(VH_DISPATCH(dt, run_im2col, xin, col, (int)d.B, (int)d.C, (int)HP, (int)WP, (int)d.KH, (int)d.KW,
                     (int)d.SH, (int)d.SW, (int)d.HO, (int)d.WO, st));
  const int vec = dt == VH_BF16 ? 8 : 4;
  const bool vok = (CKK % vec) == 0;
  p.args.a = Operand{w, (int)CKK, (int)d.O, vok && aligned16(w)};
  p.args.b = Operand{col, (int)CKK, (int)M, vok};
  return run_igemm(p, (float*)at(ws, o_g), st);
}

// Im2col backward: dcol = dY_2d . W (MatMulGradFn, matmul.rs:450-460) kept in
// fp32 in the GEMM's own [C*kh*kw][positions] layout, then col2im
// (conv.rs:1242-1298) and the pad crop in one gather kernel; dW = dY_2d^T . col
// (matmul.rs:563-574) over a re-materialised col.
static int im2col_bwd(int dt, const void* dy, const void* x, const void* w, void* dx, void* dw,
                      const ConvDims& d, hipStream_t st, size_t* need = nullptr) {
  const long HP = d.H + 2 * d.PH, WP = d.W + 2 * d.PW, CKK = d.C * d.KH * d.KW;
  const long M = d.B * d.HO * d.WO;
  VH_TRY(check_sizes({M * CKK, d.B * d.C * HP * WP}));
  const int es = elem_size(dt);
  const bool padded = d.PH || d.PW;
  // dY viewed as a [positions][O] matrix through a 1x1 "conv" gather.
  ConvGeom g1 = make_geom((int)d.B, (int)d.O, (int)d.HO, (int)d.WO, 1, 1, 1, (int)d.HO, (int)d.WO, 1, 1, 0, 0);
  ConvGeom gw = geom_of(d);
  IgemmPlan pd{}, pw{};
  size_t ws_w = 0;
  if (dx) {
    pd.dtype = dt;
    pd.akind = KD_DENSE_MN;
    pd.bkind = KD_CONV_FWD_X;
    pd.okind = OK_DENSE_T;  // launched with splits = 1 and an fp32 partial store, see below
    pd.args.M = (int)CKK;
    pd.args.N = (int)M;
    pd.args.K = (int)d.O;
    pd.args.g = g1;
    pd.args.a = Operand{w, (int)CKK, (int)CKK, 0};
    pd.args.b = Operand{dy, 0, (int)M, 0};
    pd.splits = 1;
    igemm_prepare(pd);
  }
  if (dw) {
    pw.dtype = dt;
    pw.akind = KD_CONV_WGRAD_DY;
    pw.bkind = KD_DENSE_MN;
    pw.okind = OK_DENSE;
    pw.args.M = (int)d.O;
    pw.args.N = (int)CKK;
    pw.args.K = (int)M;
    pw.args.g = gw;
    pw.args.ldd = (int)CKK;
    pw.args.d = dw;
    pw.splits = pick_splits(pw.args.M, pw.args.N, pw.args.K, dt);
    ws_w = igemm_prepare(pw);
  }
  Carve cv;
  size_t o_dcol = dx ? cv.take((size_t)M * CKK * sizeof(float)) : 0;
  size_t o_col = dw ? cv.take((size_t)M * CKK * es) : 0;
  size_t o_xp = (dw && padded) ? cv.take((size_t)d.B * d.C * HP * WP * es) : 0;
  size_t o_g = cv.take(ws_w);
  if (need) {
    *need = cv.off;
    return VH_OK;
  }
  void* ws;
  VH_TRY(ws_get(st, cv.off, &ws));
  if (dx) {
    float* dcolT = (float*)at(ws, o_dcol);
    VH_TRY(run_igemm_f32out(pd, dcolT, st));
    VH_TRY(VH_DISPATCH(dt, run_col2im_t, dcolT, dx, (int)d.B, (int)d.C, (int)d.H, (int)d.W, (int)d.KH,
                       (int)d.KW, (int)d.SH, (int)d.SW, (int)d.PH, (int)d.PW, (int)d.HO, (int)d.WO, st));
  }
  if (dw) {
    void* col = at(ws, o_col);
    const void* xin = x;
    if (padded) {
      VH_TRY(VH_DISPATCH(dt, run_pad, x, at(ws, o_xp), (int)d.B, (int)d.C, (int)d.H, (int)d.W, (int)d.PH,
                         (int)d.PW, st));
      xin = at(ws, o_xp);
    }
    VH_TRY(VH_DISPATCH(dt, run_im2col, xin, col, (int)d.B, (int)d.C, (int)HP, (int)WP, (int)d.KH, (int)d.KW,
                       (int)d.SH, (int)d.SW, (int)d.HO, (int)d.WO, st));
    pw.args.a = Operand{dy, 0, (int)d.O, aligned16(dy)};
    pw.args.b = Operand{col, (int)CKK, (int)CKK, 0};
    VH_TRY(run_igemm(pw, (float*)at(ws, o_g), st));
  }
  return VH_OK;
}

// db non-null: the bias gradient too where the per-tap kernel applies (*db_done).
static int direct_wgrad(int dt, const void* dy, const void* x, void* dw, const ConvDims& d, hipStream_t st,
                        size_t* need = nullptr, void* db = nullptr, bool* db_done = nullptr) {
  ConvGeom g = geom_of(d);
  int slices, len;
  size_t bytes = VH_DISPATCH(dt, direct_wgrad_ws, g, &slices, &len);
  if (need) {
    *need = bytes;
    return VH_OK;
  }
  void* ws;
  VH_TRY(ws_get(st, bytes, &ws));
  return VH_DISPATCH(dt, run_direct_wgrad, dy, x, dw, g, (float*)ws, slices, len, st, db, db_done);
}


// ------------------------------------------------------------------ GEMM entry helper
// bf16 products on the dense kernel: either operand may be stored with its
// contraction index contiguous (KD_DENSE_K) or its row index contiguous
// (KD_DENSE_MN: stored [K][rows], read by transposing LDS reads).  Returns
// VH_ERR_UNSUPPORTED when the shapes or alignments do not fit.
static int dense_bf16(int ak, int bk, const void* a, int lda, const void* b, int ldb, void* c, int ldc, long M,
                      long N, long K, const void* bias, hipStream_t st, void* colsum = nullptr) {
  const bool at = ak == KD_DENSE_MN, bt = bk == KD_DENSE_MN;
  if (!dense_bf16_ok(M, N, K, at, lda, bt, ldb, ldc, a, b, c)) return VH_ERR_UNSUPPORTED;
  // a grid of few tiles over a long K: the split-K implicit GEMM fills the chip instead
  if (((M + 127) / 128) * ((N + 127) / 128) < 64 && K > 2048) return VH_ERR_UNSUPPORTED;
  return dense_bf16_gemm(a, lda, at, b, ldb, bt, c, ldc, (int)M, (int)N, (int)K, bias, st, colsum);
}

// Linear's dX and dW (K-major x K-major, MN-major x MN-major) as one launch of
// the dense kernel when both take its 128 x 128 tiles: each grid alone would
// hold one block per CU.  VH_ERR_UNSUPPORTED: run them separately.
static int dense_bf16_pair(const DenseProblem& p0, const DenseProblem& p1, hipStream_t st) {
  for (const DenseProblem* p : {&p0, &p1}) {
    if (std::max({(long)p->M * p->K, (long)p->K * p->N, (long)p->M * p->N}) > kMaxElems) return VH_ERR_UNSUPPORTED;
    if (!dense_bf16_ok(p->M, p->N, p->K, p->at, p->lda, p->bt, p->ldb, p->ldc, p->a, p->b, p->c))
      return VH_ERR_UNSUPPORTED;
    if (((p->M + 127L) / 128) * ((p->N + 127L) / 128) < 64 && p->K > 2048) return VH_ERR_UNSUPPORTED;
  }
  return dense_bf16_gemm_pair(p0, p1, st);
}

static int dense_f32_pair(const DenseProblem& p0, const DenseProblem& p1, hipStream_t st) {
  for (const DenseProblem* p : {&p0, &p1}) {
    if (std::max({(long)p->M * p->K, (long)p->K * p->N, (long)p->M * p->N}) > kMaxElems) return VH_ERR_UNSUPPORTED;
    if (!dense_f32_ok(p->M, p->N, p->K, p->at, p->lda, p->bt, p->ldb, p->ldc, p->a, p->b, p->c))
      return VH_ERR_UNSUPPORTED;
  }
  return dense_f32_gemm_pair(p0, p1, st);
}

static int dense_f32(int ak, int bk, const void* a, int lda, const void* b, int ldb, void* c, int ldc, long M,
                     long N, long K, const void* bias, hipStream_t st) {
  const bool at = ak == KD_DENSE_MN, bt = bk == KD_DENSE_MN;
  if (!dense_f32_ok(M, N, K, at, lda, bt, ldb, ldc, a, b, c)) return VH_ERR_UNSUPPORTED;
  // a grid of few tiles over a long K: the split-K implicit GEMM fills the chip instead
  if (((M + 63) / 64) * ((N + 127) / 128) < 128 && K > 1024) return VH_ERR_UNSUPPORTED;
  return dense_f32_gemm(a, lda, at, b, ldb, bt, c, ldc, (int)M, (int)N, (int)K, bias, st);
}

static int gemm(int dt, int ak, int bk, const void* a, int lda, const void* b, int ldb, void* c, int ldc,
                long M, long N, long K, const void* bias, int bias_mode, hipStream_t st) {
  VH_TRY(check_sizes({M * K, K * N, M * N}));
  if (dt == VH_BF16 && g_fast_paths && (bias == nullptr || bias_mode == 2)) {
    int r = dense_bf16(ak, bk, a, lda, b, ldb, c, ldc, M, N, K, bias, st);
    if (r != VH_ERR_UNSUPPORTED) return r;
  }
  if (dt == VH_F32 && g_fast_paths && (bias == nullptr || bias_mode == 2)) {
    int r = dense_f32(ak, bk, a, lda, b, ldb, c, ldc, M, N, K, bias, st);
    if (r != VH_ERR_UNSUPPORTED) return r;
  }
  IgemmPlan p{};
  p.dtype = dt;
  p.akind = ak;
  p.bkind = bk;
  p.okind = OK_DENSE;
  p.args.M = (int)M;
  p.args.N = (int)N;
  p.args.K = (int)K;
  const int vec = dt == VH_BF16 ? 8 : 4;
  p.args.a = Operand{a, lda, (int)M, (lda % vec) == 0 && aligned16(a)};
  p.args.b = Operand{b, ldb, (int)N, (ldb % vec) == 0 && aligned16(b)};
  p.args.d = c;
  p.args.ldd = ldc;
  p.args.bias = bias;
  p.args.bias_mode = bias ? bias_mode : 0;
  p.splits = pick_splits((int)M, (int)N, (int)K, dt);
  size_t bytes = igemm_prepare(p);
  void* ws;
  VH_TRY(ws_get(st, bytes, &ws));
  return run_igemm(p, (float*)ws, st);
}

}  // namespace vh

using namespace vh;

#define VH_ENTRY()              \
  do {                          \
    int _i = ensure_init();     \
    if (_i != VH_OK) return _i; \
  } while (0)

static hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

extern "C" {

int vh_init(void) { return ensure_init(); }

int vh_set_kernel_policy(int policy) {
  if (policy != VH_POLICY_FASTEST && policy != VH_POLICY_GENERIC)
    return set_error(VH_ERR_BAD_ARG, "unknown kernel policy %d", policy);
  g_fast_paths = policy == VH_POLICY_FASTEST;
  return VH_OK;
}

const char* vh_last_error(void) { return g_err; }

int vh_alloc(size_t bytes, void** dptr) {
  VH_ENTRY();
  if (!dptr) return set_error(VH_ERR_BAD_ARG, "null output pointer");
  size_t nb = round_bytes(std::max<size_t>(bytes, 1));
  {
    std::lock_guard<std::mutex> lk(g_pool.mu);
    auto it = g_pool.free_list.find(nb);
    if (it != g_pool.free_list.end()) {
      *dptr = it->second;
      g_pool.free_list.erase(it);
      g_pool.cached--;
      g_pool.live[*dptr] = nb;
      return VH_OK;
    }
  }
  void* p = nullptr;
  if (hipMalloc(&p, nb) != hipSuccess) {
    // drop the pooled free buffers (not the workspaces: captured graphs may use them) and retry once
    (void)hipGetLastError();
    {
      std::lock_guard<std::mutex> lk(g_pool.mu);
      for (auto& kv : g_pool.free_list) (void)hipFree(kv.second);
      g_pool.free_list.clear();
      g_pool.cached = 0;
    }
    if (hipMalloc(&p, nb) != hipSuccess) {
      (void)hipGetLastError();
      return set_error(VH_ERR_OOM, "hipMalloc(%zu) failed", nb);
    }
  }
  std::lock_guard<std::mutex> lk(g_pool.mu);
  g_pool.live[p] = nb;
  *dptr = p;
  return VH_OK;
}

int vh_free(void* dptr) {
  if (!dptr) return VH_OK;
  std::lock_guard<std::mutex> lk(g_pool.mu);
  auto it = g_pool.live.find(dptr);
  if (it == g_pool.live.end()) return set_error(VH_ERR_BAD_ARG, "pointer not allocated by vh_alloc");
  size_t nb = it->second;
  g_pool.live.erase(it);
  if (nb <= kPoolMaxBytes && g_pool.cached < kPoolMaxCount && g_pool.free_list.count(nb) < 8) {
    g_pool.free_list.emplace(nb, dptr);
    g_pool.cached++;
    return VH_OK;
  }
  VH_HIP_CHECK(hipFree(dptr));
  return VH_OK;
}

int vh_release_cache(void) {
  VH_ENTRY();
  // The device, not each stream: a stream seen earlier may have been destroyed.
  VH_HIP_CHECK(hipDeviceSynchronize());
  {
    std::lock_guard<std::mutex> lk(g_pool.mu);
    for (auto& kv : g_pool.free_list) (void)hipFree(kv.second);
    g_pool.free_list.clear();
    g_pool.cached = 0;
  }
  std::lock_guard<std::mutex> lk(g_ws_mu);
  for (auto& kv : g_ws)
    if (kv.second.ptr) (void)hipFree(kv.second.ptr);
  g_ws.clear();
  for (void* p : g_ws_retired) (void)hipFree(p);
  g_ws_retired.clear();
  return VH_OK;
}

int vh_workspace_info(void* stream, void** ptr, size_t* bytes, size_t* retired) {
  std::lock_guard<std::mutex> lk(g_ws_mu);
  auto it = g_ws.find(S(stream));
  if (ptr) *ptr = it == g_ws.end() ? nullptr : it->second.ptr;
  if (bytes) *bytes = it == g_ws.end() ? 0 : it->second.bytes;
  if (retired) *retired = g_ws_retired.size();
  return VH_OK;
}

int vh_upload(void* dst, const void* src, size_t bytes, void* stream) {
  VH_ENTRY();
  if (!bytes) return VH_OK;
  if (!dst || !src) return set_error(VH_ERR_BAD_ARG, "null pointer");
  VH_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, S(stream)));
  VH_HIP_CHECK(hipStreamSynchronize(S(stream)));
  return VH_OK;
}

int vh_download(void* dst, const void* src, size_t bytes, void* stream) {
  VH_ENTRY();
  if (!bytes) return VH_OK;
  if (!dst || !src) return set_error(VH_ERR_BAD_ARG, "null pointer");
  VH_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, S(stream)));
  VH_HIP_CHECK(hipStreamSynchronize(S(stream)));
  return VH_OK;
}

int vh_stream_sync(void* stream) {
  VH_ENTRY();
  VH_HIP_CHECK(hipStreamSynchronize(S(stream)));
  return VH_OK;
}

// ------------------------------------------------------------------ matmul family
int vh_matmul(int dtype, const void* a, const void* b, void* c, int64_t m, int64_t k, int64_t n, void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  if (m < 0 || k < 0 || n < 0) return set_error(VH_ERR_BAD_SHAPE, "negative matmul dimension");
  if (m * n == 0) return VH_OK;
  if (!a || !b || !c) return set_error(VH_ERR_BAD_ARG, "null pointer");
  return gemm(dtype, KD_DENSE_K, KD_DENSE_MN, a, (int)k, b, (int)n, c, (int)n, m, n, k, nullptr, 0, S(stream));
}

int vh_matmul_backward_a(int dtype, const void* grad, const void* b, void* grad_a, int64_t m, int64_t k,
                         int64_t n, void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  if (m < 0 || k < 0 || n < 0) return set_error(VH_ERR_BAD_SHAPE, "negative matmul dimension");
  if (m * k == 0) return VH_OK;
  if (!grad || !b || !grad_a) return set_error(VH_ERR_BAD_ARG, "null pointer");
  return gemm(dtype, KD_DENSE_K, KD_DENSE_K, grad, (int)n, b, (int)n, grad_a, (int)k, m, k, n, nullptr, 0,
              S(stream));
}

int vh_matmul_backward_b(int dtype, const void* a, const void* grad, void* grad_b, int64_t m, int64_t k,
                         int64_t n, void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  if (m < 0 || k < 0 || n < 0) return set_error(VH_ERR_BAD_SHAPE, "negative matmul dimension");
  if (k * n == 0) return VH_OK;
  if (!a || !grad || !grad_b) return set_error(VH_ERR_BAD_ARG, "null pointer");
  return gemm(dtype, KD_DENSE_MN, KD_DENSE_MN, a, (int)k, grad, (int)n, grad_b, (int)n, k, n, m, nullptr, 0,
              S(stream));
}

// ------------------------------------------------------------------ im2col / col2im
int vh_im2col(int dtype, const void* input, void* col, int64_t batch, int64_t channels, int64_t height,
              int64_t width, int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w,
              int64_t h_out, int64_t w_out, void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  ConvDims d{batch, channels, 1, height, width, kernel_h, kernel_w, stride_h, stride_w, 0, 0, h_out, w_out};
  VH_TRY(check_conv(d, true));
  VH_TRY(check_sizes({batch * h_out * w_out * channels * kernel_h * kernel_w}));
  if (!input || !col) return set_error(VH_ERR_BAD_ARG, "null pointer");
  return VH_DISPATCH(dtype, run_im2col, input, col, (int)batch, (int)channels, (int)height, (int)width,
                     (int)kernel_h, (int)kernel_w, (int)stride_h, (int)stride_w, (int)h_out, (int)w_out, S(stream));
}

int vh_col2im(int dtype, const void* col, void* output, int64_t batch, int64_t channels, int64_t height,
              int64_t width, int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w,
              int64_t h_out, int64_t w_out, void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  ConvDims d{batch, channels, 1, height, width, kernel_h, kernel_w, stride_h, stride_w, 0, 0, h_out, w_out};
  VH_TRY(check_conv(d, true));
  VH_TRY(check_sizes({batch * h_out * w_out * channels * kernel_h * kernel_w}));
  if (!col || !output) return set_error(VH_ERR_BAD_ARG, "null pointer");
  return VH_DISPATCH(dtype, run_col2im, col, output, (int)batch, (int)channels, (int)height, (int)width,
                     (int)kernel_h, (int)kernel_w, (int)stride_h, (int)stride_w, (int)h_out, (int)w_out, S(stream));
}

// ------------------------------------------------------------------ conv kernels
#define VH_CONV_PROLOGUE(p0, p1, p2)                                                                        \
  VH_ENTRY();                                                                                               \
  VH_TRY(check_dtype(dtype));                                                                               \
  ConvDims d{batch, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w, pad_h, \
             pad_w, h_out, w_out};                                                                          \
  VH_TRY(check_conv(d, true));                                                                              \
  if (batch == 0) return VH_OK;                                                                             \
  if (!(p0) || !(p1) || !(p2)) return set_error(VH_ERR_BAD_ARG, "null pointer");

#define VH_CONV_ARGS                                                                                       \
  int64_t batch, int64_t in_channels, int64_t out_channels, int64_t height, int64_t width, int64_t kernel_h, \
      int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t h_out,   \
      int64_t w_out, void* stream

int vh_direct_conv(int dtype, const void* input, const void* weight, void* output, VH_CONV_ARGS) {
  VH_CONV_PROLOGUE(input, weight, output);
  ConvGeom g = geom_of(d);
  return VH_DISPATCH(dtype, run_direct_fwd, input, weight, nullptr, output, g, S(stream));
}

int vh_igemm(int dtype, const void* input, const void* weight, void* output, VH_CONV_ARGS) {
  VH_CONV_PROLOGUE(input, weight, output);
  return igemm_fwd(dtype, input, weight, nullptr, output, d, S(stream));
}

int vh_conv_backward_input(int dtype, const void* out_grad, const void* weight, void* grad_input, VH_CONV_ARGS) {
  VH_CONV_PROLOGUE(out_grad, weight, grad_input);
  ConvGeom g = geom_of(d);
  return VH_DISPATCH(dtype, run_direct_dgrad, out_grad, weight, grad_input, g, S(stream));
}

int vh_conv_backward_weight(int dtype, const void* out_grad, const void* input, void* grad_weight, VH_CONV_ARGS) {
  VH_CONV_PROLOGUE(out_grad, input, grad_weight);
  return direct_wgrad(dtype, out_grad, input, grad_weight, d, S(stream));
}

int vh_igemm_backward_input(int dtype, const void* out_grad, const void* weight, void* grad_input, VH_CONV_ARGS) {
  VH_CONV_PROLOGUE(out_grad, weight, grad_input);
  return igemm_dgrad(dtype, out_grad, weight, grad_input, d, S(stream));
}

int vh_igemm_backward_weight(int dtype, const void* out_grad, const void* input, void* grad_weight, VH_CONV_ARGS) {
  VH_CONV_PROLOGUE(out_grad, input, grad_weight);
  return igemm_wgrad(dtype, out_grad, input, grad_weight, nullptr, nullptr, d, S(stream));
}

// ------------------------------------------------------------------ algorithm selection
int vh_conv_algo_auto_select(int64_t batch, int64_t channels, int64_t height, int64_t width, int64_t kernel_size,
                             int has_gpu) {
  // conv.rs:29-69 (stride 1 / no padding assumed by the reference's estimate)
  if (height < kernel_size || width < kernel_size) return -1;
  const int64_t e = batch * (height - kernel_size + 1) * (width - kernel_size + 1) * channels * kernel_size *
                    kernel_size;
  if (has_gpu) return e > 1000000 ? VH_ALGO_IGEMM : VH_ALGO_IM2COL;
  if (e > 5000000) return VH_ALGO_DIRECT;
  if (kernel_size <= 3 && batch <= 4) return VH_ALGO_DIRECT;
  if (e > 1000000) return VH_ALGO_IGEMM;
  return VH_ALGO_IM2COL;
}

int vh_conv_algo_select_mi355x(int64_t batch, int64_t in_channels, int64_t out_channels, int64_t height,
                               int64_t width, int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                               int64_t stride_w, int64_t pad_h, int64_t pad_w) {
  (void)batch; (void)height; (void)width; (void)stride_h; (void)stride_w; (void)pad_h; (void)pad_w;
  // A reduction of <= 16 terms per output (e.g. a 3x3 kernel over 1 channel)
  // cannot feed a 16-deep MFMA step; the direct kernel streams x once instead.
  // Everything else runs as implicit GEMM on MFMA.  Im2col is never chosen
  // automatically: it writes and re-reads a C*kh*kw-times larger matrix.
  if (in_channels * kernel_h * kernel_w <= 16 || out_channels < 4) return VH_ALGO_DIRECT;
  return VH_ALGO_IGEMM;
}

// ------------------------------------------------------------------ allocating forms
// The reference's gpu_* functions allocate their result (GpuBuffer::zeros,
// kernels.rs:1133, 1233, 1333) and return it (gpu_ops.rs:160-168).  These take
// the output buffer from the pool (vh_alloc: the caller releases it with
// vh_free), run the out-parameter entry point into it, and return it in *out;
// on failure nothing is returned and the buffer goes back to the pool.
}  // extern "C"
template <typename F>
static int with_alloc(void** out, long elems, int dtype, F&& fn) {
  if (!out) return set_error(VH_ERR_BAD_ARG, "null output pointer");
  *out = nullptr;
  VH_TRY(check_dtype(dtype));
  if (elems < 0) return set_error(VH_ERR_BAD_SHAPE, "negative output size");
  void* p = nullptr;
  VH_TRY(vh_alloc((size_t)elems * elem_size(dtype), &p));
  const int st = fn(p);
  if (st != VH_OK) {
    (void)vh_free(p);
    return st;
  }
  *out = p;
  return VH_OK;
}
extern "C" {

int vh_matmul_alloc(int dtype, const void* a, const void* b, void** c, int64_t m, int64_t k, int64_t n,
                    void* stream) {
  return with_alloc(c, (long)m * n, dtype, [&](void* o) { return vh_matmul(dtype, a, b, o, m, k, n, stream); });
}

int vh_matmul_backward_a_alloc(int dtype, const void* grad, const void* b, void** grad_a, int64_t m, int64_t k,
                               int64_t n, void* stream) {
  return with_alloc(grad_a, (long)m * k, dtype,
                    [&](void* o) { return vh_matmul_backward_a(dtype, grad, b, o, m, k, n, stream); });
}

int vh_matmul_backward_b_alloc(int dtype, const void* a, const void* grad, void** grad_b, int64_t m, int64_t k,
                               int64_t n, void* stream) {
  return with_alloc(grad_b, (long)k * n, dtype,
                    [&](void* o) { return vh_matmul_backward_b(dtype, a, grad, o, m, k, n, stream); });
}

int vh_im2col_alloc(int dtype, const void* input, void** col, int64_t batch, int64_t channels, int64_t height,
                    int64_t width, int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w,
                    int64_t h_out, int64_t w_out, void* stream) {
  return with_alloc(col, (long)batch * h_out * w_out * channels * kernel_h * kernel_w, dtype, [&](void* o) {
    return vh_im2col(dtype, input, o, batch, channels, height, width, kernel_h, kernel_w, stride_h, stride_w, h_out,
                     w_out, stream);
  });
}

int vh_col2im_alloc(int dtype, const void* col, void** output, int64_t batch, int64_t channels, int64_t height,
                    int64_t width, int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w,
                    int64_t h_out, int64_t w_out, void* stream) {
  return with_alloc(output, (long)batch * channels * height * width, dtype, [&](void* o) {
    return vh_col2im(dtype, col, o, batch, channels, height, width, kernel_h, kernel_w, stride_h, stride_w, h_out,
                     w_out, stream);
  });
}

#define VH_CONV_ALLOC(NAME, ELEMS)                                                                             \
  int NAME##_alloc(int dtype, const void* t0, const void* t1, void** out, VH_CONV_ARGS) {                      \
    return with_alloc(out, (long)(ELEMS), dtype, [&](void* o) {                                                \
      return NAME(dtype, t0, t1, o, batch, in_channels, out_channels, height, width, kernel_h, kernel_w,        \
                  stride_h, stride_w, pad_h, pad_w, h_out, w_out, stream);                                      \
    });                                                                                                        \
  }
VH_CONV_ALLOC(vh_direct_conv, batch * out_channels * h_out * w_out)
VH_CONV_ALLOC(vh_igemm, batch * out_channels * h_out * w_out)
VH_CONV_ALLOC(vh_conv_backward_input, batch * in_channels * height * width)
VH_CONV_ALLOC(vh_igemm_backward_input, batch * in_channels * height * width)
VH_CONV_ALLOC(vh_conv_backward_weight, out_channels * in_channels * kernel_h * kernel_w)
VH_CONV_ALLOC(vh_igemm_backward_weight, out_channels * in_channels * kernel_h * kernel_w)
#undef VH_CONV_ALLOC

// ------------------------------------------------------------------ layers
#define VH_LAYER_ARGS                                                                                      \
  int64_t batch, int64_t in_channels, int64_t out_channels, int64_t height, int64_t width, int64_t kernel_h, \
      int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w

static int layer_dims(ConvDims& d) {
  long ho, wo;
  VH_TRY(conv_out_dim(d.H, d.KH, d.SH, d.PH, &ho));
  VH_TRY(conv_out_dim(d.W, d.KW, d.SW, d.PW, &wo));
  d.HO = ho;
  d.WO = wo;
  return check_conv(d, true);
}

static int conv2d_forward_impl(int dtype, int algo, const void* input, const void* weight, const void* bias,
                               void* output, VH_LAYER_ARGS, int* algo_used, void* stream, int act) {
  VH_TRY(check_dtype(dtype));
  ConvDims d{batch, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w,
             pad_h, pad_w, 0, 0};
  VH_TRY(layer_dims(d));
  if (algo == VH_ALGO_AUTO)
    algo = vh_conv_algo_select_mi355x(batch, in_channels, out_channels, height, width, kernel_h, kernel_w,
                                      stride_h, stride_w, pad_h, pad_w);
  if (algo < VH_ALGO_DIRECT || algo > VH_ALGO_IGEMM) return set_error(VH_ERR_BAD_ARG, "bad algorithm %d", algo);
  if (algo_used) *algo_used = algo;
  if (batch == 0) return VH_OK;
  if (!input || !weight || !output) return set_error(VH_ERR_BAD_ARG, "null pointer");
  hipStream_t st = S(stream);
  if (algo == VH_ALGO_IGEMM) return igemm_fwd(dtype, input, weight, bias, output, d, st, act);
  if (algo == VH_ALGO_IM2COL) {
    VH_TRY(im2col_fwd(dtype, input, weight, bias, output, d, st));
  } else {
    ConvGeom g = geom_of(d);
    return VH_DISPATCH(dtype, run_direct_fwd, input, weight, bias, output, g, st, act);  // ReLU fused
  }
  return act ? relu_after(dtype, output, d.B * d.O * d.HO * d.WO, st) : VH_OK;
}

int vh_conv2d_forward(int dtype, int algo, const void* input, const void* weight, const void* bias, void* output,
                      VH_LAYER_ARGS, int* algo_used, void* stream) {
  VH_ENTRY();
  return conv2d_forward_impl(dtype, algo, input, weight, bias, output, batch, in_channels, out_channels, height,
                             width, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w, algo_used, stream, 0);
}

int vh_conv2d_forward_relu(int dtype, int algo, const void* input, const void* weight, const void* bias,
                           void* output, VH_LAYER_ARGS, int* algo_used, void* stream) {
  VH_ENTRY();
  return conv2d_forward_impl(dtype, algo, input, weight, bias, output, batch, in_channels, out_channels, height,
                             width, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w, algo_used, stream, 1);
}

// need != nullptr: sizing mode -- stores the largest workspace request of the
// passes the call would run and launches nothing.
static int conv2d_backward_impl(int dtype, int algo, const void* out_grad, const void* input, const void* weight,
                                void* grad_input, void* grad_weight, void* grad_bias, VH_LAYER_ARGS, void* stream,
                                bool relu_input, size_t* need = nullptr) {
  VH_TRY(check_dtype(dtype));
  ConvDims d{batch, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w,
             pad_h, pad_w, 0, 0};
  VH_TRY(layer_dims(d));
  if (algo < VH_ALGO_DIRECT || algo > VH_ALGO_IGEMM) return set_error(VH_ERR_BAD_ARG, "bad algorithm %d", algo);
  hipStream_t st = S(stream);
  if (batch == 0) return VH_OK;
  if (!out_grad || (grad_input && !weight) || (grad_weight && !input) || (relu_input && grad_input && !input))
    return set_error(VH_ERR_BAD_ARG, "null pointer");
  const void* mask = relu_input && grad_input ? input : nullptr;
  if (need) {
    size_t most = 0, n = 0;
    auto take = [&](int r) {
      if (r == VH_OK) most = std::max(most, n);
      n = 0;
      return r;
    };
    if (algo == VH_ALGO_IM2COL) {
      if (grad_input || grad_weight)
        VH_TRY(take(im2col_bwd(dtype, out_grad, input, weight, grad_input, grad_weight, d, st, &n)));
    } else if (algo == VH_ALGO_IGEMM) {
      if (grad_input) VH_TRY(take(igemm_dgrad(dtype, out_grad, weight, grad_input, d, st, mask, &n)));
      if (grad_weight) VH_TRY(take(igemm_wgrad(dtype, out_grad, input, grad_weight, grad_bias, nullptr, d, st, &n)));
    } else if (grad_weight) {
      VH_TRY(take(direct_wgrad(dtype, out_grad, input, grad_weight, d, st, &n)));
    }
    if (grad_bias) VH_TRY(take(bias_grad_nchw(dtype, out_grad, grad_bias, d.B, d.O, d.HO * d.WO, st, &n)));
    *need = most;
    return VH_OK;
  }
  if (algo == VH_ALGO_IM2COL) {
    if (grad_input || grad_weight) VH_TRY(im2col_bwd(dtype, out_grad, input, weight, grad_input, grad_weight, d, st));
    if (mask) VH_TRY(mask_after(dtype, mask, grad_input, d.B * d.C * d.H * d.W, st));
  } else if (algo == VH_ALGO_IGEMM) {
    if (grad_input) VH_TRY(igemm_dgrad(dtype, out_grad, weight, grad_input, d, st, mask));
    if (grad_weight) {
      bool db_done = false;
      VH_TRY(igemm_wgrad(dtype, out_grad, input, grad_weight, grad_bias, &db_done, d, st));
      if (db_done) grad_bias = nullptr;
    }
  } else {
    ConvGeom g = geom_of(d);
    if (grad_input) VH_TRY(VH_DISPATCH(dtype, run_direct_dgrad, out_grad, weight, grad_input, g, st));
    if (mask) VH_TRY(mask_after(dtype, mask, grad_input, d.B * d.C * d.H * d.W, st));
    if (grad_weight) {
      bool db_done = false;
      VH_TRY(direct_wgrad(dtype, out_grad, input, grad_weight, d, st, nullptr, grad_bias, &db_done));
      if (db_done) grad_bias = nullptr;
    }
  }
  if (grad_bias) VH_TRY(bias_grad_nchw(dtype, out_grad, grad_bias, d.B, d.O, d.HO * d.WO, st));
  return VH_OK;
}

int vh_conv2d_backward(int dtype, int algo, const void* out_grad, const void* input, const void* weight,
                       void* grad_input, void* grad_weight, void* grad_bias, VH_LAYER_ARGS, void* stream) {
  VH_ENTRY();
  return conv2d_backward_impl(dtype, algo, out_grad, input, weight, grad_input, grad_weight, grad_bias, batch,
                              in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w,
                              pad_h, pad_w, stream, false);
}

int vh_conv2d_backward_relu(int dtype, int algo, const void* out_grad, const void* input, const void* weight,
                            void* grad_input, void* grad_weight, void* grad_bias, VH_LAYER_ARGS, void* stream) {
  VH_ENTRY();
  return conv2d_backward_impl(dtype, algo, out_grad, input, weight, grad_input, grad_weight, grad_bias, batch,
                              in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w,
                              pad_h, pad_w, stream, true);
}

int vh_conv2d_backward_noalloc(int dtype, int algo, const void* out_grad, const void* input, const void* weight,
                               void* grad_input, void* grad_weight, void* grad_bias, VH_LAYER_ARGS,
                               void* stream) {
  VH_ENTRY();
  void* sp;
  VH_TRY(scratch_ptr(&sp));
  size_t need = 0;
  VH_TRY(conv2d_backward_impl(dtype, algo, out_grad, input, weight, grad_input, grad_weight, grad_bias, batch,
                              in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w,
                              pad_h, pad_w, stream, false, &need));
  if (need > kScratchBytes)
    return set_error(VH_ERR_UNSUPPORTED,
                     "vh_conv2d_backward_noalloc: this call needs %zu bytes of scratch, above the static "
                     "maximum of %zu bytes; use vh_conv2d_backward",
                     need, kScratchBytes);
  FixedWs guard(sp, kScratchBytes);
  return conv2d_backward_impl(dtype, algo, out_grad, input, weight, grad_input, grad_weight, grad_bias, batch,
                              in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w,
                              pad_h, pad_w, stream, false);
}

static int convt_dims(ConvDims& d, long B, long CI, long CO, long H, long W, long KH, long KW, long SH, long SW,
                      long PH, long PW) {
  // The transposed conv is the input-gradient of a conv whose input is the
  // (B, CO, HO, WO) output and whose output is the (B, CI, H, W) input.
  long HO = (H - 1) * SH + KH - 2 * PH, WO = (W - 1) * SW + KW - 2 * PW;
  if (B < 0 || CI <= 0 || CO <= 0 || H <= 0 || W <= 0 || KH <= 0 || KW <= 0 || SH <= 0 || SW <= 0 || PH < 0 ||
      PW < 0 || HO <= 0 || WO <= 0)
    return set_error(VH_ERR_BAD_SHAPE, "bad ConvTranspose2d geometry");
  d = ConvDims{B, CO, CI, HO, WO, KH, KW, SH, SW, PH, PW, H, W};
  return check_conv(d, true);
}

// A ConvTranspose2d whose input is 1 x 1 with stride 1 and no padding (a
// generator's latent projection, conv_transpose.rs:356-435 with H = W = 1): each
// output position (kh, kw) receives exactly one tap, so the layer is the plain
// product y[n][co*KH*KW + kh*KW + kw] = sum_ci z[n][ci] W[ci][co][kh][kw] over
// the IOHW weight viewed as [CI][CO*KH*KW].  In conv terms (d): O = CI, C = CO,
// H x W = KH x KW, HO = WO = 1.
static bool convt_is_projection(const ConvDims& d) {
  return d.HO == 1 && d.WO == 1 && d.SH == 1 && d.SW == 1 && d.PH == 0 && d.PW == 0;
}

int vh_conv_transpose2d_forward(int dtype, const void* input, const void* weight, const void* bias, void* output,
                                VH_LAYER_ARGS, void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  ConvDims d;
  VH_TRY(convt_dims(d, batch, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w,
                    pad_h, pad_w));
  if (batch == 0) return VH_OK;
  if (!input || !weight || !output) return set_error(VH_ERR_BAD_ARG, "null pointer");
  hipStream_t st = S(stream);
  // y = dgrad(dy := x; W viewed OIHW with O = in_channels, C = out_channels) + bias
  if (g_fast_paths && convt_is_projection(d) && (dtype == VH_F32 || !bias)) {
    // the product, then the channel bias (for f32 the same single rounding as a fused add)
    const long NC = d.C * d.H * d.W;
    VH_TRY(gemm(dtype, KD_DENSE_K, KD_DENSE_MN, input, (int)d.O, weight, (int)NC, output, (int)NC, d.B, NC, d.O,
                nullptr, 0, st));
    return bias ? VH_DISPATCH(dtype, run_channel_bias_add, output, bias, d.B, (int)d.C, d.H * d.W, st) : VH_OK;
  }
  const ConvGeom gs = geom_of(d);
  if (g_fast_paths && dgrad_smallc_ok(gs))  // at most 4 output channels
    return VH_DISPATCH(dtype, run_dgrad_smallc, input, weight, bias, nullptr, output, gs, st);
  if ((d.SH > 1 || d.SW > 1) && g_fast_paths) {
    int r = dgrad_phases(dtype, input, weight, bias, output, d, st);
    if (r != VH_ERR_UNSUPPORTED) return r;
  }
  ConvGeom g = geom_of(d);
  const long RS = d.KH * d.KW;
  IgemmPlan p{};
  p.dtype = dtype;
  p.akind = KD_DENSE_K;
  p.bkind = KD_CONV_DGRAD_DY;
  p.okind = OK_NCHW;
  p.args.M = (int)d.C;
  p.args.N = (int)(d.B * d.H * d.W);
  p.args.K = (int)(RS * d.O);
  p.args.g = g;
  p.args.hwo = (int)(d.H * d.W);
  p.args.f_hwo = FastDiv((uint32_t)(d.H * d.W));
  p.args.d = output;
  p.args.bias = bias;
  p.args.bias_mode = bias ? 1 : 0;
  p.splits = pick_splits(p.args.M, p.args.N, p.args.K, dtype);
  size_t ws_gemm = igemm_prepare(p);
  Carve cv;
  size_t o_w = cv.take((size_t)d.O * d.C * RS * elem_size(dtype)), o_g = cv.take(ws_gemm);
  void* ws;
  VH_TRY(ws_get(st, cv.off, &ws));
  void* wd = at(ws, o_w);
  VH_TRY(VH_DISPATCH(dtype, run_relayout, weight, wd, (int)d.O, (int)d.C, (int)RS, 1, st));
  const int vec = dtype == VH_BF16 ? 8 : 4;
  p.args.a = Operand{wd, (int)(RS * d.O), (int)d.C, ((RS * d.O) % vec) == 0};
  p.args.b = Operand{input, 0, p.args.N, 0};
  return run_igemm(p, (float*)at(ws, o_g), st);
}

int vh_conv_transpose2d_backward(int dtype, const void* out_grad, const void* input, const void* weight,
                                 void* grad_input, void* grad_weight, void* grad_bias, VH_LAYER_ARGS,
                                 void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  ConvDims d;
  VH_TRY(convt_dims(d, batch, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w,
                    pad_h, pad_w));
  if (batch == 0) return VH_OK;
  if (!out_grad || (grad_input && !weight) || (grad_weight && !input))
    return set_error(VH_ERR_BAD_ARG, "null pointer");
  hipStream_t st = S(stream);
  // In conv terms (d): x = out_grad (C = out_channels), dy = input (O = in_channels).
  if (g_fast_paths && convt_is_projection(d)) {
    // dz = dY . W^T ([B][CO*KH*KW] . [CO*KH*KW][CI]); dW = z^T . dY
    const long NC = d.C * d.H * d.W;
    if (grad_input)
      VH_TRY(gemm(dtype, KD_DENSE_K, KD_DENSE_K, out_grad, (int)NC, weight, (int)NC, grad_input, (int)d.O, d.B, d.O,
                  NC, nullptr, 0, st));
    if (grad_weight)
      VH_TRY(gemm(dtype, KD_DENSE_MN, KD_DENSE_MN, input, (int)d.O, out_grad, (int)NC, grad_weight, (int)NC, d.O, NC,
                  d.B, nullptr, 0, st));
    if (grad_bias) VH_TRY(bias_grad_nchw(dtype, out_grad, grad_bias, d.B, d.C, d.H * d.W, st));
    return VH_OK;
  }
  if (grad_input) VH_TRY(igemm_fwd(dtype, out_grad, weight, nullptr, grad_input, d, st));
  if (grad_weight && dtype == VH_F32 && g_fast_paths) {
    // up-sampling layer to a few channels: dW (and dB) in one MFMA pass over the positions
    const ConvGeom g = geom_of(d);
    const size_t nb = convt_cell_wgrad_ws(g);
    if (nb) {
      void* ws;
      VH_TRY(ws_get(st, nb, &ws));
      const int r = convt_cell_wgrad_f32(input, out_grad, grad_weight, grad_bias, g, (float*)ws, nb, st);
      if (r == VH_OK) return VH_OK;
      if (r != VH_ERR_UNSUPPORTED) return r;
    }
  }
  if (grad_weight) VH_TRY(igemm_wgrad(dtype, input, out_grad, grad_weight, nullptr, nullptr, d, st));
  if (grad_bias) VH_TRY(bias_grad_nchw(dtype, out_grad, grad_bias, d.B, d.C, d.H * d.W, st));
  return VH_OK;
}

int vh_linear_forward(int dtype, const void* x, const void* weight, const void* bias, void* y, int64_t m,
                      int64_t in_features, int64_t out_features, void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  if (m < 0 || in_features < 0 || out_features < 0) return set_error(VH_ERR_BAD_SHAPE, "negative dimension");
  if (m * out_features == 0) return VH_OK;
  if (!x || !weight || !y) return set_error(VH_ERR_BAD_ARG, "null pointer");
  return gemm(dtype, KD_DENSE_K, KD_DENSE_MN, x, (int)in_features, weight, (int)out_features, y, (int)out_features,
              m, out_features, in_features, bias, 2, S(stream));
}

int vh_linear_backward(int dtype, const void* out_grad, const void* x, const void* weight, void* grad_x,
                       void* grad_weight, void* grad_bias, int64_t m, int64_t in_features, int64_t out_features,
                       void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  if (m < 0 || in_features < 0 || out_features < 0) return set_error(VH_ERR_BAD_SHAPE, "negative dimension");
  if (!out_grad || (grad_x && !weight) || (grad_weight && !x)) return set_error(VH_ERR_BAD_ARG, "null pointer");
  hipStream_t st = S(stream);
  if (dtype == VH_BF16 && g_fast_paths && grad_x && grad_weight && m * in_features * out_features &&
      std::max({m, in_features, out_features}) < (1L << 31)) {
    // db as the column sums of dY inside the dW tiles
    const DenseProblem dx{out_grad, (int)out_features, false, weight, (int)out_features, false,
                          grad_x, (int)in_features, (int)m, (int)in_features, (int)out_features, nullptr};
    const DenseProblem dw{x, (int)in_features, true, out_grad, (int)out_features, true,
                          grad_weight, (int)out_features, (int)in_features, (int)out_features, (int)m, grad_bias};
    const int r = dense_bf16_pair(dx, dw, st);
    if (r != VH_OK && r != VH_ERR_UNSUPPORTED) return r;
    if (r == VH_OK) grad_x = grad_weight = grad_bias = nullptr;  // all done
  }
  if (dtype == VH_F32 && g_fast_paths && grad_x && grad_weight && m * in_features * out_features &&
      std::max({m, in_features, out_features}) < (1L << 31)) {
    // the same pair in fp32 (whole 128 x 256 tiles only), db as column sums of dY
    const DenseProblem dx{out_grad, (int)out_features, false, weight, (int)out_features, false,
                          grad_x, (int)in_features, (int)m, (int)in_features, (int)out_features, nullptr};
    const DenseProblem dw{x, (int)in_features, true, out_grad, (int)out_features, true,
                          grad_weight, (int)out_features, (int)in_features, (int)out_features, (int)m, grad_bias};
    const int r = dense_f32_pair(dx, dw, st);
    if (r != VH_OK && r != VH_ERR_UNSUPPORTED) return r;
    if (r == VH_OK) grad_x = grad_weight = grad_bias = nullptr;  // all done
  }
  if (grad_x && m * in_features)
    VH_TRY(gemm(dtype, KD_DENSE_K, KD_DENSE_K, out_grad, (int)out_features, weight, (int)out_features, grad_x,
                (int)in_features, m, in_features, out_features, nullptr, 0, st));
  if (grad_weight && grad_bias && dtype == VH_BF16 && g_fast_paths && m * in_features * out_features &&
      std::max({m * in_features, m * out_features, in_features * out_features}) <= kMaxElems) {
    const int r = dense_bf16(KD_DENSE_MN, KD_DENSE_MN, x, (int)in_features, out_grad, (int)out_features,
                             grad_weight, (int)out_features, in_features, out_features, m, nullptr, st, grad_bias);
    if (r != VH_OK && r != VH_ERR_UNSUPPORTED) return r;
    if (r == VH_OK) grad_weight = grad_bias = nullptr;  // dW and db done
  }
  if (grad_weight && in_features * out_features)
    VH_TRY(gemm(dtype, KD_DENSE_MN, KD_DENSE_MN, x, (int)in_features, out_grad, (int)out_features, grad_weight,
                (int)out_features, in_features, out_features, m, nullptr, 0, st));
  if (grad_bias && out_features) {
    int ns, rp;
    size_t bytes = column_sum_ws((int)std::max<int64_t>(m, 1), (int)out_features, &ns, &rp);
    void* ws;
    VH_TRY(ws_get(st, bytes, &ws));
    VH_TRY(VH_DISPATCH(dtype, run_column_sum, out_grad, (int)m, (int)out_features, grad_bias, (float*)ws, ns, rp,
                       st));
  }
  return VH_OK;
}

int vh_pixel_shuffle(int dtype, const void* input, void* output, int64_t batch, int64_t channels, int64_t height,
                     int64_t width, int64_t upscale, void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  if (batch < 0 || channels <= 0 || height <= 0 || width <= 0 || upscale <= 0)
    return set_error(VH_ERR_BAD_SHAPE, "bad PixelShuffle geometry");
  VH_TRY(check_sizes({batch * channels * height * width * upscale * upscale}));
  if (batch == 0) return VH_OK;
  if (!input || !output) return set_error(VH_ERR_BAD_ARG, "null pointer");
  return VH_DISPATCH(dtype, run_pixel_shuffle, input, output, (int)batch, (int)channels, (int)height, (int)width,
                     (int)upscale, 0, S(stream));
}

int vh_pixel_shuffle_backward(int dtype, const void* out_grad, void* grad_input, int64_t batch, int64_t channels,
                              int64_t height, int64_t width, int64_t upscale, void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  if (batch < 0 || channels <= 0 || height <= 0 || width <= 0 || upscale <= 0)
    return set_error(VH_ERR_BAD_SHAPE, "bad PixelShuffle geometry");
  VH_TRY(check_sizes({batch * channels * height * width * upscale * upscale}));
  if (batch == 0) return VH_OK;
  if (!out_grad || !grad_input) return set_error(VH_ERR_BAD_ARG, "null pointer");
  return VH_DISPATCH(dtype, run_pixel_shuffle, out_grad, grad_input, (int)batch, (int)channels, (int)height,
                     (int)width, (int)upscale, 1, S(stream));
}

// ------------------------------------------------------------------ storage: casts and layouts
int vh_cast(int src_dtype, int dst_dtype, const void* src, void* dst, int64_t n, void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(src_dtype));
  VH_TRY(check_dtype(dst_dtype));
  if (n < 0) return set_error(VH_ERR_BAD_SHAPE, "negative element count");
  VH_TRY(check_sizes({(long)n}));
  if (n == 0) return VH_OK;
  if (!src || !dst) return set_error(VH_ERR_BAD_ARG, "null pointer");
  return run_cast(src_dtype, dst_dtype, src, dst, (long)n, S(stream));
}

static int layout_transform(int dtype, const void* src, void* dst, int64_t B, int64_t C, int64_t H, int64_t W,
                            bool to_nhwc, void* stream) {
  VH_TRY(check_dtype(dtype));
  if (B < 0 || C <= 0 || H <= 0 || W <= 0) return set_error(VH_ERR_BAD_SHAPE, "bad NCHW geometry");
  VH_TRY(check_sizes({(long)(B * C * H * W)}));
  if (B == 0) return VH_OK;
  if (!src || !dst || src == dst) return set_error(VH_ERR_BAD_ARG, "null or aliased pointer");
  const int R = to_nhwc ? (int)C : (int)(H * W), Cc = to_nhwc ? (int)(H * W) : (int)C;
  return VH_DISPATCH(dtype, run_batched_transpose, src, dst, (int)B, R, Cc, S(stream));
}

int vh_nchw_to_nhwc(int dtype, const void* src, void* dst, int64_t batch, int64_t channels, int64_t height,
                    int64_t width, void* stream) {
  VH_ENTRY();
  return layout_transform(dtype, src, dst, batch, channels, height, width, true, stream);
}

int vh_nhwc_to_nchw(int dtype, const void* src, void* dst, int64_t batch, int64_t channels, int64_t height,
                    int64_t width, void* stream) {
  VH_ENTRY();
  return layout_transform(dtype, src, dst, batch, channels, height, width, false, stream);
}

// ------------------------------------------------------------------ the step after dW
int vh_grad_accumulate(int dtype, void* existing, const void* new_grad, int64_t n, void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  if (n < 0) return set_error(VH_ERR_BAD_SHAPE, "negative element count");
  VH_TRY(check_sizes({(long)n}));
  if (n == 0) return VH_OK;
  if (!existing || !new_grad) return set_error(VH_ERR_BAD_ARG, "null pointer");
  return VH_DISPATCH(dtype, run_add_inplace, existing, new_grad, (long)n, S(stream));
}

int vh_optimizer_step(int op, float lr, float beta1, float beta2, float t, float eps, float weight_decay,
                      float* params, const float* grads, float* state1, float* state2, int64_t n, void* stream) {
  VH_ENTRY();
  if (op < VH_OPT_SGD || op > VH_OPT_ADAM) return set_error(VH_ERR_BAD_ARG, "bad optimizer op %d", op);
  if (n < 0) return set_error(VH_ERR_BAD_SHAPE, "negative element count");
  VH_TRY(check_sizes({(long)n}));
  if (n == 0) return VH_OK;
  if (!params || !grads || (op >= VH_OPT_SGD_MOMENTUM && !state1) || (op == VH_OPT_ADAM && !state2))
    return set_error(VH_ERR_BAD_ARG, "null pointer");
  return run_optimizer_step(op, lr, beta1, beta2, t, eps, weight_decay, params, grads, state1, state2, (long)n,
                            S(stream));
}

// ------------------------------------------------------------------ glue of the config graphs
int vh_unary(int dtype, int op, const void* input, void* output, int64_t n, void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  if (op != VH_UNARY_RELU) return set_error(VH_ERR_UNSUPPORTED, "unary op %d: only ReLU is on this path", op);
  if (n < 0) return set_error(VH_ERR_BAD_SHAPE, "negative element count");
  VH_TRY(check_sizes({(long)n}));
  if (n == 0) return VH_OK;
  if (!input || !output) return set_error(VH_ERR_BAD_ARG, "null pointer");
  return VH_DISPATCH(dtype, run_relu, input, nullptr, output, (long)n, S(stream));
}

int vh_unary_backward(int dtype, int op, const void* out_grad, const void* input, void* grad_input, int64_t n,
                      void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  if (op != VH_UNARY_RELU) return set_error(VH_ERR_UNSUPPORTED, "unary op %d: only ReLU is on this path", op);
  if (n < 0) return set_error(VH_ERR_BAD_SHAPE, "negative element count");
  VH_TRY(check_sizes({(long)n}));
  if (n == 0) return VH_OK;
  if (!out_grad || !input || !grad_input) return set_error(VH_ERR_BAD_ARG, "null pointer");
  return VH_DISPATCH(dtype, run_relu, input, out_grad, grad_input, (long)n, S(stream));
}

int vh_sum_reduce(int dtype, const void* input, int64_t n, float* result, void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  if (n < 0) return set_error(VH_ERR_BAD_SHAPE, "negative element count");
  VH_TRY(check_sizes({(long)n}));
  if (!input && n > 0) return set_error(VH_ERR_BAD_ARG, "null pointer");
  if (!result) return set_error(VH_ERR_BAD_ARG, "null pointer");
  hipStream_t st = S(stream);
  void* ws;
  VH_TRY(ws_get(st, sum_ws_bytes((long)n), &ws));
  return VH_DISPATCH(dtype, run_sum, input, (long)n, result, (float*)ws, st);
}

int vh_sum_backward(int dtype, float grad, void* grad_input, int64_t n, void* stream) {
  VH_ENTRY();
  VH_TRY(check_dtype(dtype));
  if (n < 0) return set_error(VH_ERR_BAD_SHAPE, "negative element count");
  VH_TRY(check_sizes({(long)n}));
  if (n == 0) return VH_OK;
  if (!grad_input) return set_error(VH_ERR_BAD_ARG, "null pointer");
  return VH_DISPATCH(dtype, run_fill, grad_input, (long)n, grad, S(stream));
}

}  // extern "C"
