// vh_gemm.hip -- instantiations and host dispatch of the MFMA implicit GEMM.
#include <algorithm>
#include <type_traits>

#include "vh_kernels.hpp"

namespace vh {

ConvGeom make_geom(int N, int C, int H, int W, int O, int R, int S, int P, int Q, int sh, int sw, int ph,
                   int pw) {
  ConvGeom g;
  g.N = N; g.C = C; g.H = H; g.W = W; g.O = O; g.R = R; g.S = S; g.P = P; g.Q = Q;
  g.sh = sh; g.sw = sw; g.ph = ph; g.pw = pw;
  g.fPQ = FastDiv((uint32_t)std::max(1, P * Q));
  g.fQ = FastDiv((uint32_t)std::max(1, Q));
  g.fHW = FastDiv((uint32_t)std::max(1, H * W));
  g.fW = FastDiv((uint32_t)std::max(1, W));
  g.fC = FastDiv((uint32_t)std::max(1, C));
  g.fO = FastDiv((uint32_t)std::max(1, O));
  g.fS = FastDiv((uint32_t)std::max(1, S));
  return g;
}

namespace {

template <typename T> constexpr int bk_for() { return Elem<T>::vec == 8 ? 32 : 16; }

struct Tile {
  int bm, bn;
};

// nphase: launches of several stride phases at once multiply the grid
Tile pick_tile(int M, int N, int dtype = VH_F32, int nphase = 1, int wide = 0) {
  Tile t{128, 128};
  // fp32 weight gradients: the gathers of 128 x 128 tiles feed four times the
  // MFMAs of 64 x 64 ones; split K fills the grid
  if (wide && dtype == VH_F32 && M >= 128 && N >= 128) return t;
  if (M <= 64) t.bm = 64;
  // f32 (16x16 MFMA tiles) also has 32-row tiles: a 32-channel output would
  // leave half of a 64-row tile empty
  if (M <= 32 && dtype == VH_F32) t.bm = 32;
  if (N <= 64) t.bn = 64;
  // f32 blocks are latency-bound with one block per CU: narrower tiles when the
  // wide ones would not give every CU two blocks (then lower ones, where those do)
  auto grid = [&](int bm, int bn) { return (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn) * std::max(1, nphase); };
  if (dtype == VH_F32 && t.bn == 128 && grid(t.bm, 128) < 512) t.bn = 64;
  if (dtype == VH_F32 && t.bm == 128 && grid(128, t.bn) < 512 && grid(64, t.bn) >= 512) t.bm = 64;
  return t;
}

template <typename T, int AK, int BKIND, int OUT, int BM, int BN, int BK = bk_for<T>()>
int launch_tile(IgemmPlan& p, float* ws, hipStream_t st) {
  IgemmArgs a = p.args;
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  dim3 grid((unsigned)tiles, (unsigned)std::max(1, a.nphase), (unsigned)p.splits);
  if (p.f32_out) {  // fp32 row-major result, one split
    IgemmArgs pa = a;
    pa.d = ws;
    igemm_kernel<T, AK, BKIND, OK_PARTIAL, BM, BN, BK><<<dim3((unsigned)tiles, 1, 1), 256, 0, st>>>(pa);
    VH_LAUNCH_CHECK();
    return VH_OK;
  }
  if (p.splits > 1) {
    IgemmArgs pa = a;
    pa.d = ws;
    igemm_kernel<T, AK, BKIND, OK_PARTIAL, BM, BN, BK><<<grid, 256, 0, st>>>(pa);
    VH_LAUNCH_CHECK();
    // few splits of a large weight gradient: the coalesced OIHW reduction
    if (OUT == OK_WGRAD_OIHW && a.bias_mode == 0 && a.act == 0 && a.wg_rs <= 64 && p.splits <= 8 &&
        (long)a.wg_c * a.wg_rs + (a.dbias ? 1 : 0) == a.N) {
      splitk_reduce_oihw_kernel<T><<<dim3((unsigned)a.M, (unsigned)((a.wg_c + 63) / 64)), 256,
                                     (size_t)a.wg_rs * 65 * sizeof(float), st>>>(a, ws, p.splits);
    } else {
      splitk_reduce_kernel<T, OUT><<<reduce_splits_grid((long)a.M * a.N), 256, 0, st>>>(a, ws, p.splits);
    }
    VH_LAUNCH_CHECK();
  } else {
    igemm_kernel<T, AK, BKIND, OUT, BM, BN, BK><<<grid, 256, 0, st>>>(a);
    VH_LAUNCH_CHECK();
  }
  return VH_OK;
}

template <typename T, int AK, int BKIND, int OUT>
int launch_kinds(IgemmPlan& p, float* ws, hipStream_t st) {
  Tile t = pick_tile(p.args.M, p.args.N, std::is_same<T, float>::value ? VH_F32 : VH_BF16, p.args.nphase, p.wide);
  if constexpr (std::is_same<T, float>::value) {
    // 32-row tiles take 32-deep K steps so that all 256 threads have a load unit
    if (t.bm == 32 && t.bn == 128) return launch_tile<T, AK, BKIND, OUT, 32, 128, 32>(p, ws, st);
    if (t.bm == 32) return launch_tile<T, AK, BKIND, OUT, 32, 64, 32>(p, ws, st);
  }
  if (t.bm == 128 && t.bn == 128) return launch_tile<T, AK, BKIND, OUT, 128, 128>(p, ws, st);
  if (t.bm == 64 && t.bn == 128) return launch_tile<T, AK, BKIND, OUT, 64, 128>(p, ws, st);
  if (t.bm == 128 && t.bn == 64) return launch_tile<T, AK, BKIND, OUT, 128, 64>(p, ws, st);
  return launch_tile<T, AK, BKIND, OUT, 64, 64>(p, ws, st);
}

template <typename T>
int launch_typed(IgemmPlan& p, float* ws, hipStream_t st) {
#define VH_COMBO(A, B, O)                                          \
  if (p.akind == A && p.bkind == B && p.okind == O) return launch_kinds<T, A, B, O>(p, ws, st);
  VH_COMBO(KD_DENSE_K, KD_DENSE_MN, OK_DENSE)            // matmul, Linear forward
  VH_COMBO(KD_DENSE_K, KD_DENSE_K, OK_DENSE)             // matmul backward A
  VH_COMBO(KD_DENSE_MN, KD_DENSE_MN, OK_DENSE)           // matmul backward B
  VH_COMBO(KD_DENSE_K, KD_CONV_FWD_X, OK_NCHW)           // conv fwd, convT dX
  VH_COMBO(KD_DENSE_K, KD_CONV_DGRAD_DY, OK_NCHW)        // conv dgrad, convT fwd
  VH_COMBO(KD_DENSE_K, KD_CONV_DGRAD_DY, OK_NCHW_SUB)    // the same, one stride phase at a time
  VH_COMBO(KD_CONV_WGRAD_DY, KD_CONV_WGRAD_X, OK_WGRAD_OIHW)  // conv wgrad, convT dW
  VH_COMBO(KD_DENSE_K, KD_DENSE_K, OK_NCHW)              // im2col conv fwd
  VH_COMBO(KD_DENSE_MN, KD_CONV_FWD_X, OK_DENSE_T)       // im2col conv dcol
  VH_COMBO(KD_CONV_WGRAD_DY, KD_DENSE_MN, OK_DENSE)      // im2col conv dW
#undef VH_COMBO
  return set_error(VH_ERR_BAD_ARG, "unsupported implicit-GEMM operand combination %d/%d/%d", p.akind,
                   p.bkind, p.okind);
}

}  // namespace

int pick_splits(int M, int N, int K, int dtype, int wide) {
  Tile t = pick_tile(M, N, dtype, 1, wide);
  const int bk = dtype == VH_BF16 ? 32 : 16;
  long tiles = (long)((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
  // Split K only when the tile grid leaves most of the 256 CUs idle and K is
  // long: partial sums cost 2 x splits x M x N x 4 bytes of HBM traffic.
  if (tiles >= 192 || K < 1024) return 1;
  long want = (512 + tiles - 1) / tiles;
  long maxk = std::max<long>(1, K / (bk * 8));
  return (int)std::max<long>(1, std::min<long>(std::min(want, maxk), 256));
}

size_t igemm_prepare(IgemmPlan& p) {
  const int bk = p.dtype == VH_BF16 ? 32 : 16;
  int splits = std::max(1, p.splits);
  int K = std::max(1, p.args.K);
  int chunk = (K + splits - 1) / splits;
  chunk = (chunk + bk - 1) / bk * bk;
  p.args.k_chunk = chunk;
  p.splits = (K + chunk - 1) / chunk;
  return p.splits > 1 ? (size_t)p.splits * p.args.M * p.args.N * sizeof(float) : 0;
}

int run_igemm_f32out(IgemmPlan& p, float* out, hipStream_t st) {
  if (p.args.M <= 0 || p.args.N <= 0) return VH_OK;
  p.splits = 1;
  p.args.k_chunk = p.args.K;
  p.f32_out = 1;
  int r = p.dtype == VH_BF16 ? launch_typed<bf16>(p, out, st) : launch_typed<float>(p, out, st);
  p.f32_out = 0;
  return r;
}

int run_igemm(IgemmPlan& p, float* ws, hipStream_t st) {
  if (p.args.M <= 0 || p.args.N <= 0) return VH_OK;
  if (p.dtype == VH_BF16) return launch_typed<bf16>(p, ws, st);
  return launch_typed<float>(p, ws, st);
}

}  // namespace vh
