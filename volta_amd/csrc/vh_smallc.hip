// vh_smallc.hip -- bf16 stride-1 convolution forward for layers with few input
// channels (C*R*S <= 128, e.g. an RGB first layer 3 -> 64 5x5), on gfx950 MFMA
// (v_mfma_f32_32x32x16_bf16), fp32 accumulation.
//
// The halo kernel packs K as (tap, 16-channel group): with C = 3 each group
// holds 13 zero channels and 81 % of its MFMA work is on zeros.  Here K is the
// weight's own (c, r, s) order, padded only to the next multiple of 16
// (3 x 5 x 5 = 75 -> 80).  GEMM view as in the halo kernel: rows = output
// channels o, columns = output positions m = (n, p, q), a block owns 64 o x 256
// consecutive positions (4 waves of 64 x 64); it runs TPB such position tiles of
// one output-channel tile in a row, loading the weights once.
//
// LDS per block: the weights [64 o][K] (K contiguous: each A fragment is one
// ds_read_b128), the block's input rows for all C channels with their zero
// padding ([c][ext row][padded column]), and the LDS offset of every k = (c, r,
// s) within that halo.  A lane's B fragment (8 consecutive k of its position)
// is gathered with 8 two-byte LDS reads at (position cell + offset of k); the
// halo is read from HBM once per block.  The output tile is stored through LDS
// as runs of 8 positions (16 bytes) per lane when P*Q % 8 == 0.
#include "vh_kernels.hpp"

namespace vh {

namespace {

struct SmallcArgs {
  const uint16_t* x;     // [N][C][H][W]
  const uint16_t* w;     // [O][C][R][S] = [O][K]
  const uint16_t* bias;  // [O] or nullptr
  uint16_t* y;           // [N][O][P][Q]
  int N, C, H, W, O, R, S, P, Q, ph, pw;
  int K;                 // C*R*S
  int Hp, Wp;            // padded rows per image (H + 2 ph = P + R - 1), padded columns (W + 2 pw)
  int M;                 // N*P*Q
  int rows_max;          // max ext rows any block needs
  int tiles_m, tiles_o;
  int tpb;               // position tiles per block
  int act;               // 0 none, 1 ReLU
  int vec_epi;           // 16-byte stores of 8 positions (P*Q % 8 == 0, 16-byte aligned y)
  int wpl, col0;         // halo row pitch in LDS and LDS column of padded column 0
  int vec_halo;          // halo rows as 16-byte chunks (W % 8 == 0, 16-byte aligned x), prefetched a tile ahead
  int nch;               // 16-byte chunks of one tile's halo (vec_halo)
  FastDiv fPQ, fQ, fHp, fRS, fS, fWp, fRows, fWc;
};

constexpr int kEP = 72;  // epilogue LDS pitch (elements) of a wave's 64 x 64 tile

// VEC: the 16-byte halo loads and the 16-byte epilogue (the configs' shapes),
// compiled without the element-wise paths: 157 registers, three waves per SIMD
// (with the element-wise paths in the same instance: 255, two).
template <int KP, bool VEC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(VEC ? 3 : 2))) void conv_smallc_fwd_bf16_kernel(
    SmallcArgs a) {
  const bool vec_halo = VEC || a.vec_halo, vec_epi = VEC || a.vec_epi;
  constexpr int WPITCH = KP + 8;  // weight row pitch (elements): 16-byte aligned rows, shifted banks
  extern __shared__ __attribute__((aligned(16))) uint16_t sm[];
  uint16_t* wl = sm;                                              // [64][WPITCH]
  int* koff = reinterpret_cast<int*>(sm + 64 * WPITCH);           // [KP]
  const int nh = a.C * a.rows_max * a.wpl;                         // halo elements (real channels)
  float* bl = reinterpret_cast<float*>(koff + KP);                // [64] fp32 bias of the o tile
  uint16_t* xl = reinterpret_cast<uint16_t*>(bl + 64);            // [C + 1][rows_max][Wp], plane C zeros
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave * 64;

  // logical block -> (group of tpb position tiles, o tile)
  const int groups = (a.tiles_m + a.tpb - 1) / a.tpb;
  const int lb = xcd_block(groups * a.tiles_o);
  const int tm0 = (lb / a.tiles_o) * a.tpb, o0 = (lb % a.tiles_o) * 64;
  const int plane = a.rows_max * a.wpl;  // halo elements per channel

  // weights: [64][KP], zero for k >= K and o >= O; all loads issued before the
  // LDS stores (a load-store pair per iteration would wait out each load)
  {
    constexpr int WIT = 64 * KP / 256;
    uint16_t wv[WIT];
#pragma unroll
    for (int it = 0; it < WIT; ++it) {
      const int i = tid + it * 256, o = i / KP, k = i - o * KP;
      wv[it] = (k < a.K && o0 + o < a.O) ? a.w[(long)(o0 + o) * a.K + k] : (uint16_t)0;
    }
#pragma unroll
    for (int it = 0; it < WIT; ++it) {
      const int i = tid + it * 256, o = i / KP, k = i - o * KP;
      wl[o * WPITCH + k] = wv[it];
    }
  }
  if (tid < 64) bl[tid] = (a.bias && o0 + tid < a.O) ? bf16_to_f32(a.bias[o0 + tid]) : 0.f;
  // offset of k = (c, r, s) in the halo
  for (int k = tid; k < KP; k += 256) {
    if (k < a.K) {
      uint32_t c, rs, r, s;
      a.fRS.divmod((uint32_t)k, c, rs);
      a.fS.divmod(rs, r, s);
      koff[k] = (int)c * plane + (int)r * a.wpl + (int)s + a.col0;
    } else {
      koff[k] = a.C * plane;  // padded k: the zero plane (its weights are zero too)
    }
  }

  const int half = lane >> 5, row_l = lane & 31;
  const int PQ = a.P * a.Q;
  // first ext row of tile tm (row of its first position)
  auto first_row = [&](int tm) {
    uint32_t n_a, pq_a, p_a, q_a;
    a.fPQ.divmod((uint32_t)(tm * 256), n_a, pq_a);
    a.fQ.divmod(pq_a, p_a, q_a);
    return (int)n_a * a.Hp + (int)p_a;
  };
  // vector halo: chunk i = (c, e, 8-column chunk) of the tile starting at ext
  // row es, zeros outside the image, loaded into registers and then stored
  constexpr int kHU = 4;  // chunks per lane at most
  uint4 hreg[kHU];
  int hoff[kHU];
  auto hload = [&](int es) {
#pragma unroll
    for (int u = 0; u < kHU; ++u) {
      const int i = tid + u * 256;
      hreg[u] = uint4{0u, 0u, 0u, 0u};
      hoff[u] = -1;
      if (i < a.nch) {
        uint32_t row, ch, c, e, img, hr;
        a.fWc.divmod((uint32_t)i, row, ch);
        a.fRows.divmod(row, c, e);
        a.fHp.divmod((uint32_t)(es + (int)e), img, hr);
        const int h = (int)hr - a.ph;
        hoff[u] = (int)row * a.wpl + 8 + (int)ch * 8;
        if ((int)img < a.N && h >= 0 && h < a.H)
          hreg[u] = *reinterpret_cast<const uint4*>(a.x + (((long)img * a.C + c) * a.H + h) * a.W + ch * 8);
      }
    }
  };
  const int tm_end = min(tm0 + a.tpb, a.tiles_m);
  for (int tm = tm0; tm < tm_end; ++tm) {
  const int m0 = tm * 256;
  const int e_start = first_row(tm);
  if (vec_halo) hload(e_start);  // issued before the barrier: the loads overlap the other waves' epilogue
  if (tm != tm0) __syncthreads();  // the previous tile's epilogue is done with the LDS
  if (vec_halo) {
#pragma unroll
    for (int u = 0; u < kHU; ++u)
      if (hoff[u] >= 0) *reinterpret_cast<uint4*>(xl + hoff[u]) = hreg[u];
    // the 8 columns either side of every row (the padding) are zeros
    for (int i = tid; i < a.C * a.rows_max * 2; i += 256) {
      const int row = i >> 1;
      *reinterpret_cast<uint4*>(xl + row * a.wpl + ((i & 1) ? a.W + 8 : 0)) = uint4{0u, 0u, 0u, 0u};
    }
  } else {
  // halo: ext rows e_start .. e_start + rows_max - 1 of every channel, padded
  // columns (zeros outside the image); rows past the tensor are zeros.  Element
  // i = (c, e, col) of the [C][rows_max][Wp] halo; batches of 8 loads per lane
  // are issued before their LDS stores.
  for (int base = 0; base < nh; base += 8 * 256) {
    uint16_t hv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + u * 256 + tid;
      uint16_t v = 0;
      if (i < nh) {
        uint32_t row, col, c, e, img, hr;
        a.fWp.divmod((uint32_t)i, row, col);
        a.fRows.divmod(row, c, e);
        a.fHp.divmod((uint32_t)(e_start + (int)e), img, hr);
        const int h = (int)hr - a.ph, w = (int)col - a.pw;
        if ((int)img < a.N && h >= 0 && h < a.H && w >= 0 && w < a.W)
          v = a.x[(((long)img * a.C + c) * a.H + h) * a.W + w];
      }
      hv[u] = v;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + u * 256 + tid;
      if (i < nh) xl[i] = hv[u];
    }
  }
  }
  // the zero plane (padded k), rewritten per tile: the epilogue tile overlaps it
  for (int i = tid; i < plane; i += 256) xl[nh + i] = 0;
  __syncthreads();

  // per-lane cell of each B fragment column (position) in the halo
  int bcell[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int m = m0 + wn + j * 32 + (lane & 31);
    int cidx = 0;  // positions past M read cell 0 (their results are not stored)
    if (m < a.M) {
      uint32_t n, pq, p, q;
      a.fPQ.divmod((uint32_t)m, n, pq);
      a.fQ.divmod(pq, p, q);
      cidx = ((int)n * a.Hp + (int)p - e_start) * a.wpl + (int)q;
    }
    bcell[j] = cidx;
  }

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
#pragma unroll
  for (int ks = 0; ks < KP / 16; ++ks) {
    const int kb = ks * 16 + half * 8;
    bf16x8 af[2], bfr[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const bf16x8*>(wl + (i * 32 + row_l) * WPITCH + kb);
    int ko[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) ko[e] = koff[kb + e];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint16_t v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = xl[bcell[j] + ko[e]];
      bfr[j] = __builtin_bit_cast(bf16x8, v);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
  }

  // epilogue: fp32 + bias, ReLU, one rounding
  auto val = [&](int i, int j, int v) {
    float r = acc[i][j][v] + bl[i * 32 + (v >> 2) * 8 + half * 4 + (v & 3)];
    if (a.act == 1) r = fmaxf(r, 0.f);
    return __builtin_bit_cast(uint16_t, (__bf16)r);
  };
  if (vec_epi) {
    __syncthreads();  // every wave is done with the halo and the weights
    // each wave's 64 x 64 tile goes through its own LDS region past the weights
    // and offsets, then out as 16-byte runs of 8 positions
    uint16_t* eb = xl + wave * (64 * kEP);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = i * 32 + (v >> 2) * 8 + half * 4 + (v & 3);
#pragma unroll
        for (int j = 0; j < 2; ++j) eb[row * kEP + j * 32 + row_l] = val(i, j, v);
      }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    const int k8 = lane & 7, m = m0 + wn + k8 * 8;
    uint32_t n_e, pq_e;
    a.fPQ.divmod((uint32_t)min(m, a.M - 1), n_e, pq_e);
    const long ybase = (long)n_e * a.O * PQ + pq_e;
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int row = it * 8 + (lane >> 3), o = o0 + row;
      const uint4 v = *reinterpret_cast<const uint4*>(eb + row * kEP + k8 * 8);
      if (o < a.O && m < a.M) *reinterpret_cast<uint4*>(a.y + ybase + (long)o * PQ) = v;
    }
    continue;
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int m = m0 + wn + j * 32 + row_l;
    if (m >= a.M) continue;
    uint32_t n, pq;
    a.fPQ.divmod((uint32_t)m, n, pq);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int o = o0 + i * 32 + (v >> 2) * 8 + half * 4 + (v & 3);
        if (o < a.O) a.y[((long)n * a.O + o) * PQ + pq] = val(i, j, v);
      }
  }
  }
}

// maximum ext rows spanned by a block of 256 consecutive positions
int smallc_rows_max(long M, long PQ, int Q, int Hp, int R) {
  int rm = 0;
  for (long m0 = 0; m0 < M; m0 += 256) {
    const long ml = std::min(m0 + 256, M) - 1;
    const long ra = (m0 / PQ) * Hp + (m0 % PQ) / Q, rb = (ml / PQ) * Hp + (ml % PQ) / Q;
    rm = std::max(rm, (int)(rb + R - ra));
  }
  return rm;
}

}  // namespace

int smallc_conv_bf16(const void* x, const void* w, const void* bias, void* y, int N, int C, int H, int W, int O,
                     int R, int S, int ph, int pw, int act, hipStream_t st) {
  const int K = C * R * S;
  const int P = H + 2 * ph - R + 1, Q = W + 2 * pw - S + 1;
  if (K > 128 || P <= 0 || Q <= 0 || ph > R - 1 || pw > S - 1 || act < 0 || act > 1) return VH_ERR_UNSUPPORTED;
  if ((long)N * P * Q >= (1L << 31) || (long)N * C * H * W >= (1L << 31)) return VH_ERR_UNSUPPORTED;
  SmallcArgs a{};
  a.x = (const uint16_t*)x;
  a.w = (const uint16_t*)w;
  a.bias = (const uint16_t*)bias;
  a.y = (uint16_t*)y;
  a.N = N; a.C = C; a.H = H; a.W = W; a.O = O; a.R = R; a.S = S; a.P = P; a.Q = Q; a.ph = ph; a.pw = pw;
  a.K = K;
  a.Hp = H + 2 * ph;
  a.Wp = W + 2 * pw;
  a.M = N * P * Q;
  a.act = act;
  const int KP = (K + 15) / 16 * 16;
  // the block's halo: cached per shape like the halo kernel's row-span scan is not
  // needed here (one pass over M / 256 blocks, a few thousand iterations)
  a.rows_max = smallc_rows_max(a.M, (long)P * Q, Q, a.Hp, R);
  // vector halo: rows of W + 16 elements, image column w at LDS column w + 8
  a.vec_halo = W % 8 == 0 && pw <= 8 && ((uintptr_t)x & 15) == 0 && (long)C * a.rows_max * (W / 8) <= 4 * 256;
  a.wpl = a.vec_halo ? W + 16 : a.Wp;
  a.col0 = a.vec_halo ? 8 - pw : 0;
  a.nch = a.vec_halo ? C * a.rows_max * (W / 8) : 0;
  const size_t halo = (size_t)(C + 1) * a.rows_max * a.wpl;
  a.vec_epi = ((long)P * Q) % 8 == 0 && ((uintptr_t)y & 15) == 0;
  // weights and offsets stay; the halo and the epilogue tile share the rest
  const size_t lds = (size_t)64 * (KP + 8) * 2 + (size_t)KP * 4 + 64 * 4 +
                     std::max(halo * 2, a.vec_epi ? (size_t)4 * 64 * kEP * 2 : (size_t)0);
  if (lds > 64 * 1024) return VH_ERR_UNSUPPORTED;
  a.tiles_m = (a.M + 255) / 256;
  a.tiles_o = (O + 63) / 64;
  // position tiles per block (at most 8): one round of the blocks per CU the
  // instance's registers allow on 256 CUs -- three for the vector instance, two
  // for the generic one (the weights are loaded once per block)
  const bool vec = a.vec_halo && a.vec_epi;
  const long slots = vec ? 768 : 512;
  const long tiles = (long)a.tiles_m * a.tiles_o;
  a.tpb = (int)std::max<long>(1, std::min<long>(8, (tiles + slots - 1) / slots));
  a.fPQ = FastDiv((uint32_t)(P * Q));
  a.fQ = FastDiv((uint32_t)Q);
  a.fHp = FastDiv((uint32_t)a.Hp);
  a.fRS = FastDiv((uint32_t)(R * S));
  a.fS = FastDiv((uint32_t)S);
  a.fWp = FastDiv((uint32_t)a.Wp);
  a.fRows = FastDiv((uint32_t)a.rows_max);
  a.fWc = FastDiv((uint32_t)std::max(1, W / 8));
  const dim3 grid((unsigned)((a.tiles_m + a.tpb - 1) / a.tpb * a.tiles_o));
#define VH_SMALLC_FWD(KPV)                                                    \
  if (KP == KPV) {                                                            \
    if (vec) {                                                                \
      auto kern = conv_smallc_fwd_bf16_kernel<KPV, true>;                     \
      VH_LDS_LIMIT_ONCE(kern);                                                \
      kern<<<grid, 256, lds, st>>>(a);                                        \
    } else {                                                                  \
      auto kern = conv_smallc_fwd_bf16_kernel<KPV, false>;                    \
      VH_LDS_LIMIT_ONCE(kern);                                                \
      kern<<<grid, 256, lds, st>>>(a);                                        \
    }                                                                         \
    VH_LAUNCH_CHECK();                                                        \
    return VH_OK;                                                             \
  }
  VH_SMALLC_FWD(16)
  VH_SMALLC_FWD(32)
  VH_SMALLC_FWD(48)
  VH_SMALLC_FWD(64)
  VH_SMALLC_FWD(80)
  VH_SMALLC_FWD(96)
  VH_SMALLC_FWD(112)
  VH_SMALLC_FWD(128)
#undef VH_SMALLC_FWD
  return VH_ERR_UNSUPPORTED;
}

}  // namespace vh
