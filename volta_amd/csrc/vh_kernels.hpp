// vh_kernels.hpp -- internal launch helpers of libvolta_hip (host side).
#pragma once
#include "vh_igemm.hpp"

namespace vh {

// ---- implicit GEMM (vh_gemm.hip) ----
// Describes one GEMM-shaped pass; kinds select the operand gathers and the store.
struct IgemmPlan {
  int dtype;                // VH_F32 / VH_BF16
  int akind, bkind, okind;  // OpndKind x2, OutKind
  IgemmArgs args;
  int splits;               // requested split-K factor (1 = none)
  int f32_out;              // internal: store fp32 row-major D (run_igemm_f32out)
  int wide;                 // fp32: 128 x 128 tiles (with split K) when M and N are both >= 128
};
// Fills args.k_chunk / splits and returns the fp32 workspace bytes needed.
size_t igemm_prepare(IgemmPlan& plan);
int run_igemm(IgemmPlan& plan, float* ws, hipStream_t st);
// Runs the plan with splits = 1 and stores D[M][N] row-major in fp32 to `out`.
int run_igemm_f32out(IgemmPlan& plan, float* out, hipStream_t st);
// Heuristic split-K factor for a problem with the given tile grid and K.
int pick_splits(int M, int N, int K, int dtype, int wide = 0);
ConvGeom make_geom(int N, int C, int H, int W, int O, int R, int S, int P, int Q, int sh, int sw, int ph,
                   int pw);

// ---- other kernels (vh_kernels.hip) ----
template <typename T>
int run_direct_fwd(const void* x, const void* w, const void* bias, void* y, const ConvGeom& g, hipStream_t st,
                   int act = 0);
template <typename T>
int run_col2im_t(const float* dcolT, void* x, int B, int C, int H, int W, int KH, int KW, int SH, int SW, int PH,
                 int PW, int HO, int WO, hipStream_t st);
template <typename T> int run_direct_dgrad(const void* dy, const void* w, void* dx, const ConvGeom& g, hipStream_t st);
// Input gradient for at most 4 input channels (one lane per input position; bias
// and mask optional).  VH_ERR_UNSUPPORTED when the weights exceed 16 KB of fp32.
bool dgrad_smallc_ok(const ConvGeom& g);
template <typename T>
int run_dgrad_smallc(const void* dy, const void* w, const void* bias, const void* mask, void* dx, const ConvGeom& g,
                     hipStream_t st);
// y[n][c][hw] += bias[c]
template <typename T> int run_channel_bias_add(void* y, const void* bias, long N, int C, long HW, hipStream_t st);
template <typename T> size_t direct_wgrad_ws(const ConvGeom& g, int* slices, int* slice_len);
// db non-null: the bias gradient in the same passes where the per-tap kernel
// applies (*db_done set true), else left to the caller.
template <typename T>
int run_direct_wgrad(const void* dy, const void* x, void* dw, const ConvGeom& g, float* ws, int slices,
                     int slice_len, hipStream_t st, void* db = nullptr, bool* db_done = nullptr);
template <typename T> int run_pad(const void* x, void* xp, int B, int C, int H, int W, int ph, int pw, hipStream_t st);
template <typename T> int run_crop(const void* xp, void* x, int B, int C, int H, int W, int ph, int pw, hipStream_t st);
template <typename T>
int run_im2col(const void* x, void* col, int B, int C, int H, int W, int KH, int KW, int SH, int SW, int HO,
               int WO, hipStream_t st);
template <typename T>
int run_col2im(const void* col, void* x, int B, int C, int H, int W, int KH, int KW, int SH, int SW, int HO,
               int WO, hipStream_t st);
template <typename T>
int run_relayout(const void* src, void* dst, int A, int B, int RS, int swap, hipStream_t st, int flip = 0);
// Glue: ReLU (g == nullptr) or its backward (dx = x > 0 ? g : 0); sum of n
// elements into *out (device) with a fixed order (ws: sum_ws_bytes(n)); fill.
template <typename T>
int run_relu(const void* x, const void* g, void* y, long n, hipStream_t st);
size_t sum_ws_bytes(long n);
template <typename T>
int run_sum(const void* x, long n, float* out, float* ws, hipStream_t st);
template <typename T>
int run_fill(void* y, long n, float v, hipStream_t st);
// Storage: dtype casts (f32 -> bf16 RNE) and batched transposes (out[b][c][r] = in[b][r][c]).
int run_cast(int from, int to, const void* src, void* dst, long n, hipStream_t st);
template <typename T>
int run_batched_transpose(const void* in, void* out, int B, int R, int Cc, hipStream_t st);
// The step after dW: a += b; one optimizer update (op 0 SGD, 1 SGD + momentum,
// 2 Adam) over n f32 parameters.
template <typename T>
int run_add_inplace(void* a, const void* b, long n, hipStream_t st);
int run_optimizer_step(int op, float lr, float beta1, float beta2, float t, float eps, float wd, float* param,
                       const float* grad, float* s1, float* s2, long n, hipStream_t st);
// Weights of the stride phases of an input gradient in one pass: phase p is
// dst + off[p]: [c][i][j][o] = w[o][c][kh0[p] + sh*i][kw0[p] + sw*j], i < rc[p], j < sc[p].
struct PhaseTable {
  int n;
  int kh0[16], kw0[16], rc[16], sc[16];
  long off[16];
};
template <typename T>
int run_relayout_phase(const void* w, void* dst, int O, int C, int R, int S, int sh, int sw, const PhaseTable& tab,
                       hipStream_t st);
size_t channel_sum_ws(int N, int C, int HW, int* nslice);
template <typename T>
int run_channel_sum(const void* x, int N, int C, int HW, void* out, float* ws, int nslice, hipStream_t st);
size_t column_sum_ws(int M, int N, int* nslice, int* rows_per);
template <typename T>
int run_column_sum(const void* x, int M, int N, void* out, float* ws, int nslice, int rows_per, hipStream_t st);
// out[i] = sum over z < splits of part[z][i] (fixed order), rounded once to T
template <typename T>
int run_sum_partials(const float* part, int splits, long n, void* out, hipStream_t st);
template <typename T>
int run_pixel_shuffle(const void* in, void* out, int B, int C, int H, int W, int r, int backward, hipStream_t st);

// Grouped bf16 weight layout [K/16][M][2*RS+1][8] of the halo kernels
// (vh_kernels.hip): units 2*tap and 2*tap+1 hold channels 0-7 and 8-15 of a
// 16-channel group, the last unit is zero.
int run_relayout_grouped(const void* w, void* dst, int M, int K, int RS, int mode, hipStream_t st);

// bf16 stride-1 forward for C*R*S <= 128 with K packed as (c, r, s) (vh_smallc.hip);
// act 0 none, 1 ReLU.  VH_ERR_UNSUPPORTED outside that range.
// Forward of a 4x4 stride-2 pad-1 layer with at most 4 input and 64 output
// channels (fp32; act 0 or 1 = ReLU): VH_ERR_UNSUPPORTED outside that envelope.
int cell_fwd_f32(const void* x, const void* w, const void* bias, void* y, const ConvGeom& g, int act,
                 hipStream_t st);
// Few-channel weight gradient of a 4x4 stride-2 pad-1 layer (fp32; dW and,
// when db is non-null, the bias gradient of x's channels): VH_ERR_UNSUPPORTED
// outside its envelope or when ws is smaller than convt_cell_wgrad_ws.
size_t convt_cell_wgrad_ws(const ConvGeom& g);
int convt_cell_wgrad_f32(const void* dy, const void* x, void* dw, void* db, const ConvGeom& g, float* ws,
                         size_t ws_bytes, hipStream_t st);
int smallc_conv_bf16(const void* x, const void* w, const void* bias, void* y, int N, int C, int H, int W, int O,
                     int R, int S, int ph, int pw, int act, hipStream_t st);

// ---- stride-1 bf16 halo convolution (vh_halo.hip) ----
// Computes y = conv(x, W') with C input and O output channels, where W' is
// taken from the OIHW weight w: w_mode 0 uses w as is (w is [O][C][R][S]);
// w_mode 1 uses w transposed and rotated 180 degrees (w is [C][O][R][S]: the
// input gradient of a stride-1 convolution).  ws (halo_conv_bf16_ws bytes)
// receives the grouped copy.  Returns VH_ERR_UNSUPPORTED without launching
// anything when the shape is outside the kernel's envelope.
size_t halo_conv_bf16_ws(int C, int O, int R, int S);
int halo_conv_bf16(const void* x, const void* w, int w_mode, void* ws, const void* bias, void* y, int N, int C,
                   int H, int W, int O, int R, int S, int ph, int pw, hipStream_t st, int act = 0,
                   const void* mask = nullptr);
// Most ext rows (padded input rows, R - 1 halo rows included) any block of BN
// consecutive positions spans, positions in virtual images of P x TW (PQv) over
// Hp ext rows each; Mv positions in all.  Cached per shape.
int halo_rows_max(long Mv, int BN, long PQv, int TW, int Hp, int R);

// ---- 3x3 stride-1 bf16 convolution with resident weights (vh_wres.hip) ----
// C <= 64 and O <= 64, W and the output width even; w and w_mode as for
// halo_conv_bf16 (the forward with C % 16 == 0 reads w itself, every other case
// writes the grouped copy into ws, halo_conv_bf16_ws bytes).  act 0 none,
// 1 ReLU, 2 zero where mask (laid out like y) is not positive.
// VH_ERR_UNSUPPORTED without launching outside that envelope.
int wres_conv_bf16(const void* x, const void* w, int w_mode, void* ws, const void* bias, void* y, int N, int C,
                   int H, int W, int O, int ph, int pw, hipStream_t st, int act, const void* mask);

// ---- stride-1 bf16 weight gradient (vh_wgrad.hip) ----
// Workspace bytes needed (0 if the shape is outside the kernel's envelope).
size_t wgrad_rows_ws(int N, int C, int H, int W, int O, int R, int S, int ph, int pw, bool bias);
// dW (OIHW, bf16) and optionally db; VH_ERR_UNSUPPORTED without launching if the
// shape is outside the envelope.
int wgrad_rows_bf16(const void* dy, const void* x, void* dw, void* db, int N, int C, int H, int W, int O, int R,
                    int S, int ph, int pw, float* ws, size_t ws_bytes, hipStream_t st);

// ---- fp32 3x3 stride-1 pad-1 convolutions of narrow images (vh_halo_f32.hip) ----
// Forward (dgrad = 0: w [O][C][3][3], + bias, act 1 = ReLU) or the input
// gradient as a forward conv over dY (dgrad = 1: C = the layer's O, O = the
// layer's C, w the layer's [C][O][3][3] read rotated and transposed), output
// * 1[mask > 0] when mask is given.  W % 4 == 0, W <= 28, (C, O) = (32, 64) or
// (64, 32), 16-byte aligned x and w; no workspace.
bool halo_conv3x3_f32_ok(const void* x, const void* w, int N, int C, int H, int W, int O);
int halo_conv3x3_f32(const void* x, const void* w, int dgrad, const void* bias, const void* mask, void* y, int N,
                     int C, int H, int W, int O, int act, hipStream_t st);
// Weight gradient of the same layers (dw [O][C][3][3], db [O] optional): the
// workspace bytes it needs (0: unsupported shape), and the pass (partials per
// (image, 7-row band) added in a fixed order by a second kernel).
size_t halo_wgrad3x3_f32_ws(const void* dy, const void* x, int N, int C, int H, int W, int O);
int halo_wgrad3x3_f32(const void* dy, const void* x, void* dw, void* db, int N, int C, int H, int W, int O,
                      float* ws, size_t ws_bytes, hipStream_t st);

// ---- dense bf16 products (vh_dense.hip) ----
// C[M][N] = A . B (+ bias[N] per column), bf16 in and out.  A is stored
// [M][lda] (K contiguous) or, with at, [K][lda] (M contiguous); B is stored
// [N][ldb] or, with bt, [K][ldb].
bool dense_bf16_ok(long M, long N, long K, bool at, long lda, bool bt, long ldb, long ldc, const void* a,
                   const void* b, const void* c);
// colsum (bf16 [N], optional): also the column sums of B over K, for an
// MN-major B on 128 x 128 tiles without bias (VH_ERR_UNSUPPORTED otherwise,
// before anything is queued).
int dense_bf16_gemm(const void* a, int lda, bool at, const void* b, int ldb, bool bt, void* c, int ldc, int M,
                    int N, int K, const void* bias, hipStream_t st, void* colsum = nullptr);
// Two bias-free products in one launch (each checked by dense_bf16_ok): a
// K-major A and B next to an MN-major A and B (with optional column sums of
// that B), when both run 128 x 128 tiles; VH_ERR_UNSUPPORTED otherwise (the
// caller then runs them one after the other).
struct DenseProblem {
  const void* a;
  int lda;
  bool at;
  const void* b;
  int ldb;
  bool bt;
  void* c;
  int ldc, M, N, K;
  void* colsum;
};
int dense_bf16_gemm_pair(const DenseProblem& p0, const DenseProblem& p1, hipStream_t st);
// The same in fp32 (vh_dense_f32.hip): K % 4 == 0, 16-byte aligned A and B.
bool dense_f32_ok(long M, long N, long K, bool at, long lda, bool bt, long ldb, long ldc, const void* a,
                  const void* b, const void* c);
int dense_f32_gemm(const void* a, int lda, bool at, const void* b, int ldb, bool bt, void* c, int ldc, int M,
                   int N, int K, const void* bias, hipStream_t st);
// Linear's dX and dW (+ column sums) in one launch, fp32 (each problem checked
// by dense_f32_ok); VH_ERR_UNSUPPORTED: run them separately.
int dense_f32_gemm_pair(const DenseProblem& p0, const DenseProblem& p1, hipStream_t st);

// ---- strided 1x1 bf16 convolutions, pad 0 (vh_pointwise.hip) ----
// w is the OIHW weight itself ([O][C]).  Each returns VH_ERR_UNSUPPORTED
// without launching when the shape is outside its envelope (stride >= 2;
// forward C % 16 == 0 and C <= 248, dgrad O % 16 == 0, O <= 248 and
// C % 8 == 0, wgrad stride 2, W % 8 == 0, output rows a multiple of 4).
int pw_conv_bf16_fwd(const void* x, const void* w, const void* bias, void* y, int B, int C, int H, int W, int O,
                     int S, hipStream_t st);
int pw_conv_bf16_dgrad(const void* dy, const void* w, void* dx, int B, int C, int H, int W, int O, int S,
                       hipStream_t st);
size_t pw_conv_bf16_wgrad_ws(int B, int C, int H, int W, int O, int S);
int pw_conv_bf16_wgrad(const void* dy, const void* x, void* dw, int B, int C, int H, int W, int O, int S,
                       float* ws, size_t ws_bytes, hipStream_t st);

}  // namespace vh
