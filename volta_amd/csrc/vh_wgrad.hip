// vh_wgrad.hip -- bf16 weight gradient of stride-1 convolutions on NCHW
// tensors, gfx950 MFMA (v_mfma_f32_32x32x16_bf16).
//
//   dW[o][c][r][s] = sum_{n,p,q} dY[n][o][p][q] * x[n][c][p+r-ph][q+s-pw]
//
// GEMM view: rows = o, columns = (c, tap), K = output positions.  Both operands
// are K-contiguous in NCHW memory (positions run along rows), so rows of dY and
// x are copied to LDS as they are -- no transposition.  A K step covers G
// output rows of one image; the block stages
//   * dY rows  [64 o][G][QP]       (QP = Q rounded up to 8, zero padded), and
//   * x rows   [64 c][G+R-1][XP]   (padded input columns u = w + pw),
// and every lane reads 8 consecutive positions per fragment.  Tap (r, s) of the
// x operand is row g+r, columns k+s..k+s+7: two aligned 16-byte reads and a
// byte-align funnel shift give all S horizontal taps of one row r, so x is read
// from LDS 2*R times per 16 positions instead of R*S times.
//
// Each wave accumulates a 32(o) x 32(c) x R*S tile in AGPRs.  Split-K: the grid's
// z dimension walks disjoint ranges of K steps; partial sums go to an fp32
// workspace [split][tap][O][C] (lanes store consecutive c) and a second kernel
// adds them in a fixed order and writes dW (OIHW).  Optional bias gradient
// (sum of dY over positions) is accumulated by the c-tile-0 blocks from the
// same LDS copy of dY.
#include <algorithm>

#include "vh_kernels.hpp"

namespace vh {

typedef unsigned int u32x4w __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2w __attribute__((ext_vector_type(2)));

struct WgradArgs {
  const uint16_t* dy;  // [N][O][P][Q]
  const uint16_t* x;   // [N][C][H][W]
  float* part;         // [splits][RS][O][C]
  float* dbias_part;   // [splits][O] or nullptr
  int N, C, H, W, O, P, Q, ph, pw;
  int G;               // output rows per K step
  int QP, XP;          // padded row lengths in LDS (elements)
  int OS, CS;          // LDS row strides per o / per c (elements)
  int steps_per_img;   // ceil(P / G)
  int total_steps;     // N * steps_per_img
  int steps_per_split;
  int V;               // elements per global load (8, 4 or 2): divides Q, W and the row pitch
  int cpr_dy, cpr_x;   // chunks of V elements per dY row / per x row
  int dy_bytes, x_bytes, part_bytes;  // buffer ranges (< 2^31)
};

template <int V> struct BufLoad;
template <> struct BufLoad<8> {
  __device__ static u32x4w ld(__amdgpu_buffer_rsrc_t r, int vo, int so) {
    return __builtin_bit_cast(u32x4w, __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0));
  }
};
template <> struct BufLoad<4> {
  __device__ static u32x2w ld(__amdgpu_buffer_rsrc_t r, int vo, int so) {
    return __builtin_bit_cast(u32x2w, __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, 0));
  }
};
template <> struct BufLoad<2> {
  __device__ static uint32_t ld(__amdgpu_buffer_rsrc_t r, int vo, int so) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0);
  }
};

__device__ __forceinline__ uint32_t funnel16(uint32_t lo, uint32_t hi) {
  // bytes 2..5 of (hi:lo): upper bf16 of lo, lower bf16 of hi
  return __builtin_amdgcn_alignbyte(hi, lo, 2);
}

// 8 consecutive bf16 starting s elements into the 16-element window (c0, c1)
template <int SH>
__device__ __forceinline__ u32x4w window8(const u32x4w& c0, const u32x4w& c1) {
  u32x4w r;
  if constexpr (SH == 0) {
    r = c0;
  } else if constexpr (SH == 2) {
    r = u32x4w{c0.y, c0.z, c0.w, c1.x};
  } else if constexpr (SH == 4) {
    r = u32x4w{c0.z, c0.w, c1.x, c1.y};
  } else if constexpr (SH == 6) {
    r = u32x4w{c0.w, c1.x, c1.y, c1.z};
  } else if constexpr (SH == 8) {
    r = c1;
  } else if constexpr (SH == 1) {
    r = u32x4w{funnel16(c0.x, c0.y), funnel16(c0.y, c0.z), funnel16(c0.z, c0.w), funnel16(c0.w, c1.x)};
  } else if constexpr (SH == 3) {
    r = u32x4w{funnel16(c0.y, c0.z), funnel16(c0.z, c0.w), funnel16(c0.w, c1.x), funnel16(c1.x, c1.y)};
  } else if constexpr (SH == 5) {
    r = u32x4w{funnel16(c0.z, c0.w), funnel16(c0.w, c1.x), funnel16(c1.x, c1.y), funnel16(c1.y, c1.z)};
  } else {  // 7
    r = u32x4w{funnel16(c0.w, c1.x), funnel16(c1.x, c1.y), funnel16(c1.y, c1.z), funnel16(c1.z, c1.w)};
  }
  return r;
}

template <int V>
struct VecT;
template <> struct VecT<8> { using t = u32x4w; };
template <> struct VecT<4> { using t = u32x2w; };
template <> struct VecT<2> { using t = uint32_t; };

// Stores V bf16 elements at LDS element offset `off`.  mode 0: off is V-aligned
// (one vector store); mode 1: off is even (dword stores); mode 2: off is odd
// (the odd horizontal padding case: one element, shifted pairs, one element).
template <int V>
__device__ __forceinline__ void lds_put(uint16_t* base, int off, const typename VecT<V>::t& v, int mode) {
  if (mode == 0) {
    *reinterpret_cast<typename VecT<V>::t*>(base + off) = v;
    return;
  }
  const uint32_t* d = reinterpret_cast<const uint32_t*>(&v);
  if (mode == 1) {
#pragma unroll
    for (int i = 0; i < V / 2; ++i) *reinterpret_cast<uint32_t*>(base + off + 2 * i) = d[i];
    return;
  }
  base[off] = (uint16_t)(d[0] & 0xffffu);
#pragma unroll
  for (int i = 0; i < V / 2 - 1; ++i)
    *reinterpret_cast<uint32_t*>(base + off + 1 + 2 * i) = __builtin_amdgcn_alignbyte(d[i + 1], d[i], 2);
  base[off + V - 1] = (uint16_t)(d[V / 2 - 1] >> 16);
}

template <int R, int S, int V, int ND, int NX>
__global__ __launch_bounds__(256) void wgrad_rows_bf16_kernel(WgradArgs a) {
  constexpr int RS = R * S;
  constexpr int TO = 64, TC = 64;  // block tile (o, c)
  using VT = typename VecT<V>::t;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar) index
  const int wo = (wave >> 1) * 32, wc = (wave & 1) * 32;
  const int o0 = blockIdx.x * TO, c0 = blockIdx.y * TC;
  const int split = blockIdx.z;
  const int G = a.G, QP = a.QP, XP = a.XP, OS = a.OS, CS = a.CS;
  const int XR = G + R - 1;
  const int dy_elems = TO * OS, x_elems = TC * CS;
  const int stage = dy_elems + x_elems;  // elements per stage
#define DYS(st) (smem + (st) * stage)
#define XS(st) (smem + (st) * stage + dy_elems)

  const int step_b = split * a.steps_per_split;
  const int step_e = min(a.total_steps, step_b + a.steps_per_split);
  const int nsteps = max(0, step_e - step_b);

  // zero both stages once: padding columns/rows are never written by the loader
  for (int i = tid; i < 2 * stage / 8; i += 256) reinterpret_cast<u32x4w*>(smem)[i] = u32x4w{0u, 0u, 0u, 0u};

  // Per-thread load items, fixed for the whole kernel: (row, chunk) of the dY
  // tile and of the x tile.  Only the (image, first row) base moves per step.
  const long PQ = (long)a.P * a.Q, HW = (long)a.H * a.W;
  const int dy_items = TO * G * a.cpr_dy, x_items = TC * XR * a.cpr_x;
  int dy_goff[ND], dy_loff[ND], dy_g[ND];
  int x_goff[NX], x_loff[NX], x_j[NX];
#pragma unroll
  for (int it = 0; it < ND; ++it) {
    int i = tid + it * 256;
    int ch = i % a.cpr_dy, t = i / a.cpr_dy, g = t % G, o = t / G;
    bool ok = i < dy_items && o0 + o < a.O;
    dy_g[it] = ok ? g : 1 << 20;  // invalid items never load
    dy_goff[it] = ok ? (int)(((o0 + o) * PQ + g * a.Q + ch * V) * 2) : 0;
    dy_loff[it] = i < dy_items ? o * OS + g * QP + ch * V : -1;
  }
#pragma unroll
  for (int it = 0; it < NX; ++it) {
    int i = tid + it * 256;
    int ch = i % a.cpr_x, t = i / a.cpr_x, j = t % XR, c = t / XR;
    bool ok = i < x_items && c0 + c < a.C;
    x_j[it] = ok ? j : 1 << 20;
    x_goff[it] = ok ? (int)(((c0 + c) * HW + j * a.W + ch * V) * 2) : 0;
    x_loff[it] = i < x_items ? c * CS + j * XP + a.pw + ch * V : -1;
  }
  const int x_mode = (a.pw % V) == 0 ? 0 : (a.pw % 2) == 0 ? 1 : 2;
  const __amdgpu_buffer_rsrc_t dyr = __builtin_amdgcn_make_buffer_rsrc((void*)a.dy, (short)0, a.dy_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t xrr = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.x_bytes, 0x00020000);

  VT rdy[ND], rx[NX];
  auto gload = [&](int step) {
    const int n = step / a.steps_per_img;
    const int p0 = (step - n * a.steps_per_img) * G;
    // scalar byte offsets of this step's image / first row; per-item parts are in VGPRs
    const int dys = (int)(((long)n * a.O * PQ + (long)p0 * a.Q) * 2);
    const int xso = (int)(((long)n * a.C * HW + (long)(p0 - a.ph) * a.W) * 2);
    const int gmax = a.P - p0;                           // rows g < gmax exist
    const int jmin = a.ph - p0, jmax = a.H + a.ph - p0;  // rows j in [jmin, jmax) exist
#pragma unroll
    for (int it = 0; it < ND; ++it) {
      const bool ok = dy_g[it] < gmax;
      rdy[it] = BufLoad<V>::ld(dyr, ok ? dy_goff[it] + dys : (int)0x80000000u, 0);
    }
#pragma unroll
    for (int it = 0; it < NX; ++it) {
      const bool ok = x_j[it] >= jmin && x_j[it] < jmax;
      rx[it] = BufLoad<V>::ld(xrr, ok ? x_goff[it] + xso : (int)0x80000000u, 0);
    }
  };
  auto sstore = [&](int st) {
    uint16_t* d = DYS(st);
    uint16_t* xs = XS(st);
#pragma unroll
    for (int it = 0; it < ND; ++it)
      if (dy_loff[it] >= 0) *reinterpret_cast<VT*>(d + dy_loff[it]) = rdy[it];
#pragma unroll
    for (int it = 0; it < NX; ++it)
      if (x_loff[it] >= 0) lds_put<V>(xs, x_loff[it], rx[it], x_mode);
  };

  f32x16 acc[RS];
#pragma unroll
  for (int t = 0; t < RS; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[t][v] = 0.f;
  float dbias = 0.f;
  const bool do_bias = a.dbias_part != nullptr && blockIdx.y == 0;

  const int nchunk = G * (QP >> 3);  // even by construction
  const int grp = lane >> 5, rl = lane & 31;

  __syncthreads();
  if (nsteps > 0) {
    gload(step_b);
    sstore(0);
  }
  __syncthreads();
  for (int ks = 0; ks < nsteps; ++ks) {
    const int st = ks & 1;
    if (ks + 1 < nsteps) gload(step_b + ks + 1);
    const uint16_t* dl = DYS(st) + (wo + rl) * OS;
    const uint16_t* xl = XS(st) + (wc + rl) * CS;
    // this lane group's chunk t = kk + grp as (row g, column k0); rows hold QP/8 chunks
    int g = 0, k0 = grp * 8;
    if (k0 >= QP) {
      k0 -= QP;
      g = 1;
    }
    for (int kk = 0; kk < nchunk; kk += 2) {
      const bf16x8 af = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4w*>(dl + g * QP + k0));
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint16_t* xr = xl + (g + r) * XP + k0;
        const u32x4w c0v = *reinterpret_cast<const u32x4w*>(xr);
        const u32x4w c1v = *reinterpret_cast<const u32x4w*>(xr + 8);
#pragma unroll
        for (int s = 0; s < S; ++s) {
          u32x4w wv;
          if (s == 0) wv = window8<0>(c0v, c1v);
          else if (s == 1) wv = window8<1>(c0v, c1v);
          else if (s == 2) wv = window8<2>(c0v, c1v);
          else if (s == 3) wv = window8<3>(c0v, c1v);
          else wv = window8<4>(c0v, c1v);
          acc[r * S + s] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, __builtin_bit_cast(bf16x8, wv),
                                                                    acc[r * S + s], 0, 0, 0);
        }
      }
      k0 += 16;
      while (k0 >= QP) {  // QP = 8 advances two rows per 16 positions
        k0 -= QP;
        ++g;
      }
    }
    if (do_bias) {
      // thread t sums quarter (t % 4) of dY row o = t / 4 of this stage
      const int o = tid >> 2, part = tid & 3;
      const uint16_t* drow = DYS(st) + o * OS;
      const int len = G * QP, q4 = len >> 2, beg = part * q4, end = part == 3 ? len : beg + q4;
      for (int k = beg; k < end; ++k) dbias += bf16_to_f32(drow[k]);
    }
    if (ks + 1 < nsteps) sstore(st ^ 1);
    __syncthreads();
  }
#undef DYS
#undef XS

  // partial tile store: part[split][tap][o][c], lanes walk c.  Per-lane offset:
  // column c and the half-wave's 4-row shift; scalar offset: (split, tap, row).
  {
    const __amdgpu_buffer_rsrc_t pr =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.part, (short)0, a.part_bytes, 0x00020000);
    const int c = c0 + wc + rl;
    const int ohalf = (lane >> 5) * 4;
    const int voff = c < a.C ? (ohalf * a.C + c) * 4 : (int)0x80000000u;
#pragma unroll
    for (int t = 0; t < RS; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int orow = o0 + wo + (v >> 2) * 8 + (v & 3);
        if (orow + ohalf < a.O)
        {
          const float val = acc[t][v];  // (a bit_cast of the vector element itself reads element 0)
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val), pr, voff,
                                                (((split * RS + t) * a.O) + orow) * a.C * 4, 0);
        }
      }
  }
  if (do_bias) {
    // combine the 4 quarter sums of each o (adjacent lanes)
    dbias += __shfl_xor(dbias, 1, 64);
    dbias += __shfl_xor(dbias, 2, 64);
    const int o = o0 + (tid >> 2);
    if ((tid & 3) == 0 && o < a.O) a.dbias_part[(long)split * a.O + o] = dbias;
  }
}

// dW[o][c][tap] = sum_z part[z][tap][o][c], bf16 out.  16 lanes share one output
// element: lane g adds the splits z = g, g+16, ... and the 16 partial sums are
// combined in a fixed butterfly order, so the result does not depend on timing.
__global__ __launch_bounds__(256) void wgrad_reduce_bf16_kernel(const float* __restrict__ part, int splits,
                                                                int RS, int O, int C, uint16_t* __restrict__ dw) {
  const long total = (long)RS * O * C;
  const int g = threadIdx.x & 15;
  const long i = (long)blockIdx.x * 16 + (threadIdx.x >> 4);
  float s = 0.f;
  if (i < total)
    for (int z = g; z < splits; z += 16) s += part[(long)z * total + i];
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if (g == 0 && i < total) {
    int c = (int)(i % C);
    long t = i / C;
    int o = (int)(t % O);
    int tap = (int)(t / O);
    dw[((long)o * C + c) * RS + tap] = f32_to_bf16(s);
  }
}

__global__ __launch_bounds__(256) void bias_reduce_bf16_kernel(const float* __restrict__ part, int splits, int O,
                                                               uint16_t* __restrict__ db) {
  int o = blockIdx.x * 256 + threadIdx.x;
  if (o >= O) return;
  float s = 0.f;
  for (int z = 0; z < splits; ++z) s += part[(long)z * O + o];
  db[o] = f32_to_bf16(s);
}

namespace {

struct WgradPlan {
  WgradArgs a;
  int splits, nd, nx;
  size_t lds;
  int tiles_o, tiles_c;
};

bool plan_wgrad(WgradPlan& pl, int N, int C, int H, int W, int O, int R, int S, int ph, int pw) {
  WgradArgs& a = pl.a;
  const int P = H + 2 * ph - R + 1, Q = W + 2 * pw - S + 1;
  if (P <= 0 || Q <= 0 || R != 3 || S != 3) return false;
  a.N = N; a.C = C; a.H = H; a.W = W; a.O = O; a.P = P; a.Q = Q; a.ph = ph; a.pw = pw;
  // vector width: divides Q and W (rows start at multiples of Q / W elements)
  a.V = 8;
  while (a.V > 1 && ((Q % a.V) || (W % a.V))) a.V >>= 1;
  if (a.V < 2) return false;
  a.cpr_dy = Q / a.V;
  a.cpr_x = W / a.V;
  a.QP = (Q + 7) / 8 * 8;
  a.G = std::max(1, std::min(P, 128 / a.QP));
  // prefer a row count that divides P (no zero rows in an image's last step)
  for (int g = a.G; g * 2 > a.G && g > 1; --g)
    if (P % g == 0 && ((g * a.QP / 8) & 1) == 0) {
      a.G = g;
      break;
    }
  if (((a.G * a.QP / 8) & 1) != 0) {  // chunks per step must pair up into 16-deep MFMA steps
    if (a.G < P) a.G += 1; else a.QP += 8;
    if (((a.G * a.QP / 8) & 1) != 0) a.QP += 8;
  }
  a.XP = std::max(a.QP + 16, (W + 2 * pw + 7) / 8 * 8);
  // LDS row strides: an ODD number of 16-byte units, so the 16 lanes that one
  // LDS cycle serves (16 rows, 16 bytes each) land on 16 distinct bank groups
  a.OS = a.G * a.QP;
  if (((a.OS / 8) & 1) == 0) a.OS += 8;
  a.CS = (a.G + R - 1) * a.XP;
  if (((a.CS / 8) & 1) == 0) a.CS += 8;
  const size_t stage = (size_t)(64 * a.OS + 64 * a.CS) * 2;
  pl.lds = 2 * stage;
  if (pl.lds > 160 * 1024) return false;
  const int dy_items = 64 * a.G * a.cpr_dy, x_items = 64 * (a.G + R - 1) * a.cpr_x;
  pl.nd = (dy_items + 255) / 256;
  pl.nx = (x_items + 255) / 256;
  const int max_nd = a.V == 2 ? 16 : 8, max_nx = a.V == 2 ? 24 : 16;
  if (pl.nd > max_nd || pl.nx > max_nx) return false;
  a.steps_per_img = (P + a.G - 1) / a.G;
  a.total_steps = N * a.steps_per_img;
  pl.tiles_o = (O + 63) / 64;
  pl.tiles_c = (C + 63) / 64;
  const int tiles = pl.tiles_o * pl.tiles_c;
  // one wave of blocks over the 256 CUs (one block per CU: LDS-limited)
  int splits = std::max(1, std::min(a.total_steps, (256 + tiles - 1) / tiles));
  a.steps_per_split = (a.total_steps + splits - 1) / splits;
  pl.splits = (a.total_steps + a.steps_per_split - 1) / a.steps_per_split;
  return true;
}

template <int R, int S, int V, int ND, int NX>
int launch_wgrad(const WgradPlan& pl, hipStream_t st) {
  auto kern = wgrad_rows_bf16_kernel<R, S, V, ND, NX>;
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    attr = true;
  }
  dim3 grid((unsigned)pl.tiles_o, (unsigned)pl.tiles_c, (unsigned)pl.splits);
  kern<<<grid, 256, pl.lds, st>>>(pl.a);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <int V>
int launch_v(const WgradPlan& pl, hipStream_t st) {
  if (pl.nd <= 4 && pl.nx <= 8) return launch_wgrad<3, 3, V, 4, 8>(pl, st);
  if (pl.nd <= 8 && pl.nx <= 16) return launch_wgrad<3, 3, V, 8, 16>(pl, st);
  if constexpr (V == 2) return launch_wgrad<3, 3, V, 16, 24>(pl, st);
  return VH_ERR_UNSUPPORTED;
}

}  // namespace

size_t wgrad_rows_ws(int N, int C, int H, int W, int O, int R, int S, int ph, int pw, bool bias) {
  WgradPlan pl;
  if (!plan_wgrad(pl, N, C, H, W, O, R, S, ph, pw)) return 0;
  size_t b = (size_t)pl.splits * R * S * O * C * sizeof(float);
  if (bias) b += (size_t)pl.splits * O * sizeof(float) + 256;
  return b;
}

int wgrad_rows_bf16(const void* dy, const void* x, void* dw, void* db, int N, int C, int H, int W, int O, int R,
                    int S, int ph, int pw, float* ws, size_t ws_bytes, hipStream_t st) {
  WgradPlan pl;
  if (!plan_wgrad(pl, N, C, H, W, O, R, S, ph, pw)) return VH_ERR_UNSUPPORTED;
  const size_t need = wgrad_rows_ws(N, C, H, W, O, R, S, ph, pw, db != nullptr);
  if (need > ws_bytes) return set_error(VH_ERR_BAD_ARG, "wgrad workspace too small");
  {
    const long dyb = (long)N * O * pl.a.P * pl.a.Q * 2, xb = (long)N * C * H * W * 2;
    const long pb = (long)pl.splits * R * S * O * C * 4;
    if (dyb >= (1L << 31) - 16 || xb >= (1L << 31) - 16 || pb >= (1L << 31) - 16) return VH_ERR_UNSUPPORTED;
    pl.a.dy_bytes = (int)dyb;
    pl.a.x_bytes = (int)xb;
    pl.a.part_bytes = (int)pb;
  }
  pl.a.dy = (const uint16_t*)dy;
  pl.a.x = (const uint16_t*)x;
  pl.a.part = ws;
  const size_t pbytes = (size_t)pl.splits * R * S * O * C * sizeof(float);
  pl.a.dbias_part = db ? (float*)((char*)ws + ((pbytes + 255) & ~size_t(255))) : nullptr;
  int rc = pl.a.V == 8 ? launch_v<8>(pl, st) : pl.a.V == 4 ? launch_v<4>(pl, st) : launch_v<2>(pl, st);
  if (rc) return rc;
  const long total = (long)R * S * O * C;
  wgrad_reduce_bf16_kernel<<<(int)((total + 15) / 16), 256, 0, st>>>(ws, pl.splits, R * S, O, C, (uint16_t*)dw);
  VH_LAUNCH_CHECK();
  if (db) {
    bias_reduce_bf16_kernel<<<(O + 255) / 256, 256, 0, st>>>(pl.a.dbias_part, pl.splits, O, (uint16_t*)db);
    VH_LAUNCH_CHECK();
  }
  return VH_OK;
}

}  // namespace vh
