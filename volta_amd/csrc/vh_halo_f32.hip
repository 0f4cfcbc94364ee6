// vh_halo_f32.hip -- fp32 3x3 stride-1 pad-1 convolutions of narrow images
// (W <= 28, e.g. 28 x 28 feature maps) on gfx950 MFMA (v_mfma_f32_16x16x4f32).
//
// Forward:        y[n][o][p][q] = sum_{c,r,s} x[n][c][p+r-1][q+s-1] w[o][c][r][s]   (+ bias, ReLU)
// Input gradient: the same form over dY with the weights rotated by 180 degrees
// and O / C swapped, dx[n][c][p][q] = sum_{o,r,s} dY[n][o][p+r-1][q+s-1] w[o][c][2-r][2-s],
// then dx * 1[mask > 0] for a fused ReLU backward.
//
// GEMM view of a block: rows = output channels (<= 64), columns = 7 output
// rows x 32 columns of one image (a row's columns q >= W are computed and
// dropped), K = (c, r, s) in the weight's own order.  A block stages the whole
// weight matrix and the 9 input rows its outputs read in LDS:
//   weights  wl[kq][o][k']        k = kq * K/4 + k'  (the MFMA's four k lanes each walk one quarter of K)
//   input    xs[kq][c'][row][36]  channel kq * C/4 + c'; image column w at 4 + w, zeros at 3 and past W
// so every tap (r, s) is an address shift, and a B fragment is one ds_read_b32
// per lane (16 consecutive columns).  The quarter strides are 16 mod 64 floats
// and the weight rows have an odd pitch (K/4 + 1): the 16 rows x four k lanes of
// a fragment read hit disjoint banks, and the staging writes of a row's
// consecutive k are consecutive words.
// Waves: (o-tile of 16, column half of 16, row group); with 64 output channels
// a wave takes all 7 rows (one A and 7 B fragments per k step), with 32 two
// waves on one SIMD take rows 0-3 and 4-6.
//
// Weight gradient: dw[o][c][r][s] = sum_{n,p,q} dy[n][o][p][q] x[n][c][p+r-1][q+s-1]
// (and db[o] = sum dy).  GEMM view of a block (image, band of 7 output rows):
// rows o, columns c for each tap, K = the band's 7 x 32 positions (columns
// q >= W hold dY = 0).  LDS: dY ds[o][7 x 32] (pitch 260 floats) and the 9
// input rows as in the forward, xs[c][9][36] (plane 324 floats); both pitches
// are 4 mod 64, so a fragment -- 16 rows x 4 consecutive positions -- is
// conflict-free.  Wave = (o-tile of 16, c-tile of 16) with the 9 tap tiles
// (36 accumulators): per k step one dY and 9 shifted x fragments.  Each block
// writes its partial sums ([tap][O][C], then [O] for the bias) to the
// workspace; a second kernel adds the blocks' partials in block order.
#include <type_traits>

#include "vh_kernels.hpp"

namespace vh {

namespace {

constexpr int kHfXP = 36;    // LDS input row pitch (floats)
constexpr int kHfRB = 7;     // output rows per block
constexpr int kHfRows = kHfRB + 2;

struct HaloF32Args {
  const float* x;     // [N][C][H][W]
  const float* w;     // forward: [O][C][3][3]; input gradient: the layer's [C][O][3][3]
  const float* bias;  // [O] or nullptr
  const float* mask;  // [N][O][H][W] or nullptr: output * 1[mask > 0]
  float* y;           // [N][O][H][W]
  int N, H, W, bands, act;
};

// floats rounded up to 16 mod 64
constexpr int quarter_stride(int n) { return n + ((16 - n % 64) % 64 + 64) % 64; }

template <int C, int O>
struct HfCfg {
  static constexpr int K = 9 * C, KQ = K / 4, CQ = C / 4;
  static constexpr int OT = O / 16, RG = 8 / (2 * OT);  // o-tiles, row groups (rows 0-3 / 4-6)
  static constexpr int WP = KQ + 1;  // weight row pitch (odd)
  static constexpr int WQS = quarter_stride(WP * O);
  static constexpr int XQS = quarter_stride(CQ * kHfRows * kHfXP);
  static constexpr int LDS_FLOATS = 4 * WQS + 4 * XQS + 64;  // + tail read by dropped columns
  static_assert(C % 4 == 0 && O % 16 == 0 && O <= 64 && RG * 2 * OT == 8 && RG <= 2, "shape");
  static_assert(kHfRB == 7, "row groups of 4 and 3");
  static_assert(LDS_FLOATS * 4 <= 160 * 1024, "LDS");
};

template <int C, int O, bool DG>
__global__ __launch_bounds__(512) void halo_f32_kernel(HaloF32Args a) {
  using Cfg = HfCfg<C, O>;
  constexpr int K = Cfg::K, KQ = Cfg::KQ, CQ = Cfg::CQ, OT = Cfg::OT, RG = Cfg::RG;
  constexpr int WQS = Cfg::WQS, XQS = Cfg::XQS, WP = Cfg::WP;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float* wl = lds;
  float* xs = lds + 4 * WQS;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = blockIdx.x / a.bands, p0 = (blockIdx.x % a.bands) * kHfRB;
  const int H = a.H, W = a.W;

  // ---- staging: all global loads first, then the LDS stores
  constexpr int WU = O * K / 4;                       // weight float4 units
  constexpr int WIT = (WU + 511) / 512;
  constexpr int XU = C * kHfRows * 9;                 // input row slots of 4 floats (9 per row)
  constexpr int XIT = (XU + 511) / 512;
  float4 wv[WIT], xv[XIT];
#pragma unroll
  for (int it = 0; it < WIT; ++it) {
    const int u = tid + it * 512;
    wv[it] = u < WU ? reinterpret_cast<const float4*>(a.w)[u] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const int wq = W / 4;
#pragma unroll
  for (int it = 0; it < XIT; ++it) {
    const int u = tid + it * 512;
    xv[it] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (u < XU) {
      const int slot = u % 9, row = (u / 9) % kHfRows, c = u / (9 * kHfRows);
      const int h = p0 - 1 + row;
      if (slot >= 1 && slot <= wq && h >= 0 && h < H)
        xv[it] = *reinterpret_cast<const float4*>(a.x + (((long)n * C + c) * H + h) * W + 4 * (slot - 1));
    }
  }
#pragma unroll
  for (int it = 0; it < WIT; ++it) {
    const int u = tid + it * 512;
    if (u < WU) {
      const float v[4] = {wv[it].x, wv[it].y, wv[it].z, wv[it].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int f = 4 * u + e;
        int i, k;
        if constexpr (DG) {  // f = (o_layer * O + c_layer) * 9 + rs -> A[c_layer][o_layer * 9 + 8 - rs]
          const int rs = f % 9, oc = f / 9;
          i = oc % O;
          k = (oc / O) * 9 + 8 - rs;
        } else {  // f = o * K + k
          i = f / K;
          k = f % K;
        }
        wl[(k / KQ) * WQS + i * WP + k % KQ] = v[e];
      }
    }
  }
#pragma unroll
  for (int it = 0; it < XIT; ++it) {
    const int u = tid + it * 512;
    if (u < XU) {
      const int slot = u % 9, rc = u / 9;  // rc = c * rows + row
      const int c = rc / kHfRows, row = rc % kHfRows;
      *reinterpret_cast<float4*>(&xs[(c / CQ) * XQS + ((c % CQ) * kHfRows + row) * kHfXP + 4 * slot]) = xv[it];
    }
  }
  __syncthreads();

  // ---- multiply and store: wave = (o-tile, column half, row group)
  const int ot = wave % OT, half = (wave / OT) & 1, rg = wave / (2 * OT);
  const int kq = lane >> 4, j = lane & 15;
  const float* ap = wl + kq * WQS + (ot * 16 + j) * WP;
  const float* bp = xs + kq * XQS + half * 16 + j + 3;
  const int q = half * 16 + j;
  auto phase = [&](auto NRV, int t0) {
    constexpr int NR = decltype(NRV)::value;
    f32x4 acc[NR];
#pragma unroll
    for (int t = 0; t < NR; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KQ; ++ks) {
      const int cc = ks / 9, r = (ks % 9) / 3, s = ks % 3;
      const float av = ap[ks];
#pragma unroll
      for (int t = 0; t < NR; ++t)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bp[(cc * kHfRows + t0 + t + r) * kHfXP + s], acc[t], 0,
                                                      0, 0);
    }
    // 16 consecutive columns of 4 output channels per store
    if (q >= W) return;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int o = ot * 16 + kq * 4 + v;
      const float b = a.bias ? a.bias[o] : 0.f;
#pragma unroll
      for (int t = 0; t < NR; ++t) {
        const int p = p0 + t0 + t;
        if (p >= H) break;
        const long off = (((long)n * O + o) * H + p) * W + q;
        float val = acc[t][v] + b;
        if (a.act == 1) val = fmaxf(val, 0.f);
        if (a.mask) val = a.mask[off] > 0.f ? val : 0.f;
        a.y[off] = val;
      }
    }
  };
  if constexpr (RG == 1) {
    phase(std::integral_constant<int, kHfRB>(), 0);
  } else {
    if (rg == 0) phase(std::integral_constant<int, 4>(), 0);
    else phase(std::integral_constant<int, 3>(), 4);
  }
}

template <int C, int O, bool DG>
int launch_halo_f32(const HaloF32Args& a, hipStream_t st) {
  auto kern = halo_f32_kernel<C, O, DG>;
  VH_LDS_LIMIT_ONCE(kern);
  kern<<<(unsigned)(a.N * a.bands), 512, (size_t)HfCfg<C, O>::LDS_FLOATS * 4, st>>>(a);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

constexpr int kHwDP = 260;  // LDS dY row pitch per output channel (7 x 32 positions + 36)
constexpr int kHwXP = kHfRows * kHfXP;  // LDS x plane per channel (324)

struct HaloWgradF32Args {
  const float* dy;  // [N][O][H][W]
  const float* x;   // [N][C][H][W]
  float* part;      // [blocks][9 * O * C + O]
  int N, H, W, bands;
};

template <int C, int O>
__global__ __launch_bounds__(512) void halo_wgrad_f32_kernel(HaloWgradF32Args a) {
  static_assert((O / 16) * (C / 16) == 8 && O % 16 == 0 && C % 16 == 0, "8 waves of 16 x 16 tiles");
  constexpr int DS_FLOATS = O * kHwDP, XS_FLOATS = C * kHwXP;
  static_assert((DS_FLOATS + XS_FLOATS + 64) * 4 <= 160 * 1024, "LDS");
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float* ds = lds;
  float* xs = lds + DS_FLOATS;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = blockIdx.x / a.bands, p0 = (blockIdx.x % a.bands) * kHfRB;
  const int H = a.H, W = a.W, wq = W / 4;

  // ---- staging: dY rows p0 .. p0+6 (8 slots of 4 per row, zeros past W and
  // H) and x rows p0-1 .. p0+7 (9 slots: image column w at 4 + w), loads first
  constexpr int DU = O * kHfRB * 8, DIT = (DU + 511) / 512;
  constexpr int XU = C * kHfRows * 9, XIT = (XU + 511) / 512;
  float4 dv[DIT], xv[XIT];
#pragma unroll
  for (int it = 0; it < DIT; ++it) {
    const int u = tid + it * 512;
    dv[it] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (u < DU) {
      const int slot = u & 7, t = (u >> 3) % kHfRB, o = (u >> 3) / kHfRB;
      const int p = p0 + t;
      if (slot < wq && p < H)
        dv[it] = *reinterpret_cast<const float4*>(a.dy + (((long)n * O + o) * H + p) * W + 4 * slot);
    }
  }
#pragma unroll
  for (int it = 0; it < XIT; ++it) {
    const int u = tid + it * 512;
    xv[it] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (u < XU) {
      const int slot = u % 9, row = (u / 9) % kHfRows, c = u / (9 * kHfRows);
      const int h = p0 - 1 + row;
      if (slot >= 1 && slot <= wq && h >= 0 && h < H)
        xv[it] = *reinterpret_cast<const float4*>(a.x + (((long)n * C + c) * H + h) * W + 4 * (slot - 1));
    }
  }
#pragma unroll
  for (int it = 0; it < DIT; ++it) {
    const int u = tid + it * 512;
    if (u < DU) {
      const int slot = u & 7, t = (u >> 3) % kHfRB, o = (u >> 3) / kHfRB;
      *reinterpret_cast<float4*>(&ds[o * kHwDP + t * 32 + 4 * slot]) = dv[it];
    }
  }
#pragma unroll
  for (int it = 0; it < XIT; ++it) {
    const int u = tid + it * 512;
    if (u < XU) {
      const int slot = u % 9, rc = u / 9;
      *reinterpret_cast<float4*>(&xs[rc * kHfXP + 4 * slot]) = xv[it];  // rc = c * 9 + row
    }
  }
  __syncthreads();

  // ---- multiply: wave = (o-tile, c-tile); lane = (row i of the fragment, position qk)
  const int ot = wave % (O / 16), ct = wave / (O / 16);
  const int i = lane & 15, qk = lane >> 4;
  const float* ap = ds + (ot * 16 + i) * kHwDP + qk;
  const float* bp = xs + (ct * 16 + i) * kHwXP + qk + 3;
  f32x4 acc[9];
#pragma unroll
  for (int rs = 0; rs < 9; ++rs) acc[rs] = f32x4{0.f, 0.f, 0.f, 0.f};
  float bsum = 0.f;  // this lane's dY sum (the bias gradient; c-tile 0 only)
#pragma unroll
  for (int t = 0; t < kHfRB; ++t)
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float av = ap[t * 32 + 4 * u];
      bsum += av;
#pragma unroll
      for (int rs = 0; rs < 9; ++rs)
        acc[rs] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bp[(t + rs / 3) * kHfXP + 4 * u + rs % 3], acc[rs], 0, 0, 0);
    }

  // ---- partial sums of this block: [tap][o][c] (16 consecutive c per store), then [o]
  float* part = a.part + (size_t)blockIdx.x * (9 * O * C + O);
#pragma unroll
  for (int rs = 0; rs < 9; ++rs)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int o = ot * 16 + 4 * qk + v;
      part[((size_t)rs * O + o) * C + ct * 16 + i] = acc[rs][v];
    }
  // the four position lanes of each o, added in lane-group order
  const float b1 = __shfl(bsum, i + 16), b2 = __shfl(bsum, i + 32), b3 = __shfl(bsum, i + 48);
  if (ct == 0 && qk == 0) part[9 * O * C + ot * 16 + i] = ((bsum + b1) + b2) + b3;
}

// dw[o][c][r][s] (+ db[o]) = the blocks' partials added in block order
template <int C, int O>
__global__ __launch_bounds__(256) void halo_wgrad_f32_reduce_kernel(const float* __restrict__ part, int blocks,
                                                                    int lg_g, float* __restrict__ dw,
                                                                    float* __restrict__ db) {
  constexpr long total = 9L * O * C + O;
  reduce_splits_vec4_block(part, blocks, total, lg_g, [&](long idx, float v) {
    if (idx < 9L * O * C) {
      const int rs = (int)(idx / (O * C)), oc = (int)(idx % (O * C));
      dw[oc * 9 + rs] = v;  // oc = o * C + c
    } else if (db) {
      db[idx - 9L * O * C] = v;
    }
  }, (int)blockIdx.x, (int)gridDim.x);
}

template <int C, int O>
int launch_halo_wgrad_f32(const HaloWgradF32Args& a, float* dw, float* db, hipStream_t st) {
  auto kern = halo_wgrad_f32_kernel<C, O>;
  VH_LDS_LIMIT_ONCE(kern);
  const int blocks = a.N * a.bands;
  kern<<<(unsigned)blocks, 512, (size_t)(O * kHwDP + C * kHwXP + 64) * 4, st>>>(a);
  VH_LAUNCH_CHECK();
  const long total = 9L * O * C + O;
  const int lg_g = reduce_vec4_lg_groups(blocks);
  halo_wgrad_f32_reduce_kernel<C, O><<<reduce_vec4_grid(total, lg_g), 256, 0, st>>>(a.part, blocks, lg_g, dw, db);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

}  // namespace

size_t halo_wgrad3x3_f32_ws(const void* dy, const void* x, int N, int C, int H, int W, int O) {
  if (!halo_conv3x3_f32_ok(x, x, N, C, H, W, O) || ((uintptr_t)dy & 15)) return 0;
  return (size_t)N * ((H + kHfRB - 1) / kHfRB) * (9 * (size_t)O * C + O) * sizeof(float);
}

int halo_wgrad3x3_f32(const void* dy, const void* x, void* dw, void* db, int N, int C, int H, int W, int O,
                      float* ws, size_t ws_bytes, hipStream_t st) {
  const size_t need = halo_wgrad3x3_f32_ws(dy, x, N, C, H, W, O);
  if (!need || need > ws_bytes || ((uintptr_t)ws & 15)) return VH_ERR_UNSUPPORTED;
  HaloWgradF32Args a{(const float*)dy, (const float*)x, ws, N, H, W, (H + kHfRB - 1) / kHfRB};
  if (C == 32 && O == 64) return launch_halo_wgrad_f32<32, 64>(a, (float*)dw, (float*)db, st);
  if (C == 64 && O == 32) return launch_halo_wgrad_f32<64, 32>(a, (float*)dw, (float*)db, st);
  return VH_ERR_UNSUPPORTED;
}

bool halo_conv3x3_f32_ok(const void* x, const void* w, int N, int C, int H, int W, int O) {
  return W % 4 == 0 && W >= 4 && W <= 28 && H >= 1 && N >= 1 && ((C == 32 && O == 64) || (C == 64 && O == 32)) &&
         (((uintptr_t)x | (uintptr_t)w) & 15) == 0 && (long)N * ((H + kHfRB - 1) / kHfRB) < (1L << 31) &&
         (long)N * std::max(C, O) * H * W < (1L << 31);
}

int halo_conv3x3_f32(const void* x, const void* w, int dgrad, const void* bias, const void* mask, void* y, int N,
                     int C, int H, int W, int O, int act, hipStream_t st) {
  if (!halo_conv3x3_f32_ok(x, w, N, C, H, W, O) || act < 0 || act > 1) return VH_ERR_UNSUPPORTED;
  const int bands = (H + kHfRB - 1) / kHfRB;
  HaloF32Args a{(const float*)x, (const float*)w, (const float*)bias, (const float*)mask, (float*)y,
                N, H, W, bands, act};
  if (C == 32 && O == 64) return dgrad ? launch_halo_f32<32, 64, true>(a, st) : launch_halo_f32<32, 64, false>(a, st);
  if (C == 64 && O == 32) return dgrad ? launch_halo_f32<64, 32, true>(a, st) : launch_halo_f32<64, 32, false>(a, st);
  return VH_ERR_UNSUPPORTED;
}

}  // namespace vh
