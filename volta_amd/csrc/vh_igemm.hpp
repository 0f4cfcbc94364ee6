// vh_igemm.hpp -- generic MFMA implicit-GEMM kernel for gfx950.
//
// One kernel template computes D[M][N] = sum_k A(row m, k) * B(row n, k) with fp32
// accumulation, where each operand is fetched by an "operand kind" (a dense
// matrix in either orientation, or one of the implicit-im2col gathers of a
// convolution pass) and the result is stored by an "output kind" (row-major,
// NCHW scatter, OIHW weight-gradient scatter, or fp32 split-K partials).
//
// Tiling: 256 threads = 4 waves (2 x 2), block tile BM x BN, K step BK.
//  * bf16: v_mfma_f32_32x32x16_bf16, wave tile (BM/2) x (BN/2) of 32x32 tiles.
//  * f32 : v_mfma_f32_16x16x4_f32,  wave tile (BM/2) x (BN/2) of 16x16 tiles.
// LDS holds both operands K-major ([row][k], 16-byte units of VEC elements, row
// pitch BK+PADK elements = 80 bytes) and is double-buffered: global loads for
// step k+1 are in flight while the MFMAs of step k run.
#pragma once
#include <type_traits>

#include "vh_common.hpp"

namespace vh {

enum OpndKind : int {
  KD_DENSE_K = 0,       // elem(r,k) = p[r*ld + k]
  KD_DENSE_MN = 1,      // elem(r,k) = p[k*ld + r]
  KD_CONV_FWD_X = 2,    // r = out position (n,p,q); k = (kh,kw,c): x[n][c][p*sh+kh-ph][q*sw+kw-pw]
  KD_CONV_DGRAD_DY = 3, // r = in position (n,h,w); k = (kh,kw,o): dy[n][o][(h+ph-kh)/sh][(w+pw-kw)/sw]
  KD_CONV_WGRAD_DY = 4, // r = o; k = out position (n,p,q): dy[n][o][p][q]
  KD_CONV_WGRAD_X = 5,  // r = (kh,kw,c); k = out position (n,p,q): x[n][c][p*sh+kh-ph][q*sw+kw-pw]
};

enum OutKind : int {
  OK_DENSE = 0,      // d[row*ldd + col]
  OK_DENSE_T = 1,    // d[col*ldd + row]
  OK_NCHW = 2,       // row = channel (M channels), col = (n, hw) over N*HWo
  OK_WGRAD_OIHW = 3, // row = o, col = (kh,kw,c) -> d[o][c][kh][kw]
  OK_PARTIAL = 4,    // fp32 ws[(z*M + row)*N + col]
  OK_NCHW_SUB = 5,   // row = channel, col = (n, hh, ww) of one stride phase (a, b) of an
                     // NCHW output: d[n][row][sub_sh*hh + sub_a][sub_sw*ww + sub_b]
};

// Convolution geometry (x: N,C,H,W; weight O,C,R,S; y: N,O,P,Q).
struct ConvGeom {
  int N, C, H, W, O, R, S, P, Q, sh, sw, ph, pw;
  FastDiv fPQ, fQ, fHW, fW, fC, fO, fS;
};

struct Operand {
  const void* p;
  int ld;      // dense leading dimension (elements)
  int rows;    // valid rows (M for A, N for B)
  int vec_ok;  // dense K-major: 16-byte vector loads allowed (aligned ld/base)
};

// One stride phase of a multi-phase launch (blockIdx.y): its A operand, the
// gather's padding and the output phase (OK_NCHW_SUB).
struct PhaseArg {
  const void* a;
  int offa, offb, sub_a, sub_b;
};

struct IgemmArgs {
  int M, N, K;
  Operand a, b;
  void* d;
  int ldd;
  const void* bias;  // same dtype as T; nullptr = none
  int bias_mode;     // 0 none, 1 per row, 2 per column
  int k_chunk;       // K range per blockIdx.z (multiple of BK)
  int hwo;           // OK_NCHW: spatial size of the output
  FastDiv f_hwo;     // OK_NCHW: divide by hwo
  FastDiv f_cw;      // OK_WGRAD_OIHW: divide by C (channels of the weight grad)
  int wg_c, wg_rs;   // OK_WGRAD_OIHW: C and R*S
  int sub_sh, sub_sw, sub_a, sub_b, sub_H, sub_W;  // OK_NCHW_SUB: strides, phase, full extents
  FastDiv f_wsub;    // OK_NCHW_SUB: divide by the phase's width
  int act;           // epilogue: 0 none, 1 ReLU, 2 zero where mask <= 0 (mask laid out like d)
  const void* mask;
  void* dbias;       // OK_WGRAD_OIHW: column wg_c*wg_rs (a B row of ones) is the bias gradient -> dbias[row]
  ConvGeom g;
  int nphase;        // > 1: blockIdx.y selects ph[blockIdx.y] (same M, N, K for every phase)
  PhaseArg ph[4];
};

// ---------------------------------------------------------------- operand loaders
// Each thread fills "units" of VEC consecutive k for one operand row.
template <typename T, int KIND>
struct Loader {
  using S = typename Elem<T>::storage;
  static constexpr int VEC = Elem<T>::vec;
  static constexpr bool kFastest =
      (KIND == KD_DENSE_K || KIND == KD_CONV_WGRAD_DY || KIND == KD_CONV_WGRAD_X);

  // per-unit row state
  int row;
  bool valid;
  bool ones;       // KD_CONV_WGRAD_X with op.ld == 1: the last row is all ones (bias column)
  int s0, s1, s2;  // kind-specific precomputed quantities
  const S* base;

  __device__ __forceinline__ void init(const Operand& op, const ConvGeom& g, int r) {
    row = r;
    valid = r < op.rows;
    ones = KIND == KD_CONV_WGRAD_X && op.ld == 1 && r == op.rows - 1;
    base = reinterpret_cast<const S*>(op.p);
    if (!valid || ones) return;
    if (KIND == KD_CONV_FWD_X) {
      uint32_t n, pq, p, q;
      g.fPQ.divmod((uint32_t)r, n, pq);
      g.fQ.divmod(pq, p, q);
      s0 = (int)p * g.sh - g.ph;
      s1 = (int)q * g.sw - g.pw;
      s2 = (int)n * g.C * g.H * g.W;
    } else if (KIND == KD_CONV_DGRAD_DY) {
      uint32_t n, hw, h, w;
      g.fHW.divmod((uint32_t)r, n, hw);
      g.fW.divmod(hw, h, w);
      s0 = (int)h + g.ph;
      s1 = (int)w + g.pw;
      s2 = (int)n * g.O * g.P * g.Q;
    } else if (KIND == KD_CONV_WGRAD_DY) {
      s0 = r * g.P * g.Q;
    } else if (KIND == KD_CONV_WGRAD_X) {
      uint32_t rs, c, kh, kw;
      g.fC.divmod((uint32_t)r, rs, c);
      g.fS.divmod(rs, kh, kw);
      s0 = (int)kh - g.ph;
      s1 = (int)kw - g.pw;
      s2 = (int)c * g.H * g.W;
    }
  }

  // Loads VEC elements for k0..k0+VEC-1 into out (zeros where out of range).
  __device__ __forceinline__ void load(const Operand& op, const ConvGeom& g, int k0, int K,
                                       S (&out)[VEC]) const {
#pragma unroll
    for (int j = 0; j < VEC; ++j) out[j] = S(0);
    if (!valid || k0 >= K) return;
    if (KIND == KD_CONV_WGRAD_X && ones) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) out[j] = k0 + j < K ? Elem<T>::from_f32(1.f) : S(0);
      return;
    }
    if (KIND == KD_DENSE_K) {
      const S* src = base + (long)row * op.ld + k0;
      if (op.vec_ok && k0 + VEC <= K) {
        *reinterpret_cast<uint4*>(out) = *reinterpret_cast<const uint4*>(src);
      } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j)
          if (k0 + j < K) out[j] = src[j];
      }
    } else if (KIND == KD_DENSE_MN) {
      const S* src = base + (long)k0 * op.ld + row;
#pragma unroll
      for (int j = 0; j < VEC; ++j)
        if (k0 + j < K) out[j] = src[(long)j * op.ld];
    } else if (KIND == KD_CONV_FWD_X) {
      const int HW = g.H * g.W;
      if ((g.C % VEC) == 0) {
        uint32_t rs, c0, kh, kw;
        g.fC.divmod((uint32_t)k0, rs, c0);
        g.fS.divmod(rs, kh, kw);
        int h = s0 + (int)kh, w = s1 + (int)kw;
        if (h >= 0 && h < g.H && w >= 0 && w < g.W) {
          const S* src = base + s2 + (int)c0 * HW + h * g.W + w;
#pragma unroll
          for (int j = 0; j < VEC; ++j) out[j] = src[j * HW];
        }
      } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          int k = k0 + j;
          if (k < K) {
            uint32_t rs, c, kh, kw;
            g.fC.divmod((uint32_t)k, rs, c);
            g.fS.divmod(rs, kh, kw);
            int h = s0 + (int)kh, w = s1 + (int)kw;
            if (h >= 0 && h < g.H && w >= 0 && w < g.W) out[j] = base[s2 + (int)c * HW + h * g.W + w];
          }
        }
      }
    } else if (KIND == KD_CONV_DGRAD_DY) {
      const int PQ = g.P * g.Q;
      if ((g.O % VEC) == 0) {
        uint32_t rs, o0, kh, kw;
        g.fO.divmod((uint32_t)k0, rs, o0);
        g.fS.divmod(rs, kh, kw);
        int t = s0 - (int)kh, u = s1 - (int)kw;
        if (t >= 0 && u >= 0) {
          // stride 1 (every stride phase is): no division
          const bool unit = g.sh == 1 && g.sw == 1;
          int p = unit ? t : t / g.sh, q = unit ? u : u / g.sw;
          if (p * g.sh == t && q * g.sw == u && p < g.P && q < g.Q) {
            const S* src = base + s2 + (int)o0 * PQ + p * g.Q + q;
#pragma unroll
            for (int j = 0; j < VEC; ++j) out[j] = src[j * PQ];
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          int k = k0 + j;
          if (k < K) {
            uint32_t rs, o, kh, kw;
            g.fO.divmod((uint32_t)k, rs, o);
            g.fS.divmod(rs, kh, kw);
            int t = s0 - (int)kh, u = s1 - (int)kw;
            if (t >= 0 && u >= 0) {
              const bool unit = g.sh == 1 && g.sw == 1;
              int p = unit ? t : t / g.sh, q = unit ? u : u / g.sw;
              if (p * g.sh == t && q * g.sw == u && p < g.P && q < g.Q)
                out[j] = base[s2 + (int)o * PQ + p * g.Q + q];
            }
          }
        }
      }
    } else if (KIND == KD_CONV_WGRAD_DY) {
      const int PQ = g.P * g.Q;
      uint32_t n, pq;
      g.fPQ.divmod((uint32_t)k0, n, pq);
      const S* src = base + (int)n * g.O * PQ + s0 + (int)pq;
      if ((PQ % VEC) == 0 && op.vec_ok && k0 + VEC <= K) {
        *reinterpret_cast<uint4*>(out) = *reinterpret_cast<const uint4*>(src);
      } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          if (k0 + j < K) {
            out[j] = src[0];
          }
          ++pq;
          ++src;
          if ((int)pq == PQ) {  // next image: skip the other channels
            pq = 0;
            src += (g.O - 1) * PQ;
          }
        }
      }
    } else if (KIND == KD_CONV_WGRAD_X) {
      uint32_t n, pq, p, q;
      g.fPQ.divmod((uint32_t)k0, n, pq);
      g.fQ.divmod(pq, p, q);
      const int HW = g.H * g.W;
      int nb = (int)n * g.C * HW + s2;
      int pi = (int)p, qi = (int)q;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        if (k0 + j < K) {
          int h = pi * g.sh + s0, w = qi * g.sw + s1;
          if (h >= 0 && h < g.H && w >= 0 && w < g.W) out[j] = base[nb + h * g.W + w];
        }
        if (++qi == g.Q) {
          qi = 0;
          if (++pi == g.P) {
            pi = 0;
            nb += g.C * HW;
          }
        }
      }
    }
  }
};

// ---------------------------------------------------------------- MFMA traits
template <typename T> struct Mma;

template <> struct Mma<bf16> {
  static constexpr int TM = 32, TN = 32, TK = 16, NACC = 16;
  using acc_t = f32x16;
  // lane l supplies row l%32, k = 8*(l/32)..+8 of the 32x16 operand slice
  __device__ static inline int frag_row(int lane) { return lane & 31; }
  __device__ static inline int frag_k(int lane) { return (lane >> 5) * 8; }
  __device__ static inline acc_t mma(const uint16_t* a, const uint16_t* b, acc_t c) {
    bf16x8 av = *reinterpret_cast<const bf16x8*>(a);
    bf16x8 bv = *reinterpret_cast<const bf16x8*>(b);
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, c, 0, 0, 0);
  }
  // accumulator register v of lane l holds (row, col) of the 32x32 tile
  __device__ static inline int acc_row(int lane, int v) { return (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3); }
  __device__ static inline int acc_col(int lane) { return lane & 31; }
};

// fp32, 32 x 32 tiles (v_mfma_f32_32x32x2_f32): for block tiles of at least
// 64 x 64; the same fragment and accumulator layout as the bf16 32 x 32 tile
struct MmaF32x32 {
  static constexpr int TM = 32, TN = 32, TK = 2, NACC = 16;
  using acc_t = f32x16;
  __device__ static inline int frag_row(int lane) { return lane & 31; }
  __device__ static inline int frag_k(int lane) { return lane >> 5; }
  __device__ static inline acc_t mma(const float* a, const float* b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(*a, *b, c, 0, 0, 0);
  }
  __device__ static inline int acc_row(int lane, int v) { return (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3); }
  __device__ static inline int acc_col(int lane) { return lane & 31; }
};

template <> struct Mma<float> {
  static constexpr int TM = 16, TN = 16, TK = 4, NACC = 4;
  using acc_t = f32x4;
  __device__ static inline int frag_row(int lane) { return lane & 15; }
  __device__ static inline int frag_k(int lane) { return lane >> 4; }
  __device__ static inline acc_t mma(const float* a, const float* b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(*a, *b, c, 0, 0, 0);
  }
  __device__ static inline int acc_row(int lane, int v) { return (lane >> 4) * 4 + v; }
  __device__ static inline int acc_col(int lane) { return lane & 15; }
};

// ---------------------------------------------------------------- output store
template <typename T, int OUT>
__device__ __forceinline__ long out_index(const IgemmArgs& args, int row, int col) {
  if (OUT == OK_DENSE) return (long)row * args.ldd + col;
  if (OUT == OK_DENSE_T) return (long)col * args.ldd + row;
  if (OUT == OK_NCHW) {
    uint32_t n, hw;
    args.f_hwo.divmod((uint32_t)col, n, hw);
    return ((long)n * args.M + row) * args.hwo + hw;
  }
  if (OUT == OK_NCHW_SUB) {
    uint32_t n, hw, hh, ww;
    args.f_hwo.divmod((uint32_t)col, n, hw);
    args.f_wsub.divmod(hw, hh, ww);
    return (((long)n * args.M + row) * args.sub_H + args.sub_sh * (int)hh + args.sub_a) * args.sub_W +
           args.sub_sw * (int)ww + args.sub_b;
  }
  uint32_t rs, c;  // OK_WGRAD_OIHW
  args.f_cw.divmod((uint32_t)col, rs, c);
  return ((long)row * args.wg_c + c) * args.wg_rs + rs;
}

// Epilogue mask (act 2): true where the mask value at the output element is positive.
template <typename T, int OUT>
__device__ __forceinline__ bool mask_keep(const IgemmArgs& args, int row, int col) {
  using S = typename Elem<T>::storage;
  if (row >= args.M || col >= args.N) return false;
  return Elem<T>::to_f32(reinterpret_cast<const S*>(args.mask)[out_index<T, OUT>(args, row, col)]) > 0.f;
}

// keep: the act-2 mask test for this element (computed by mask_keep, possibly
// ahead of earlier stores).
template <typename T, int OUT>
__device__ __forceinline__ void store_out(const IgemmArgs& args, int row, int col, float v, bool keep = true) {
  using S = typename Elem<T>::storage;
  if (row >= args.M || col >= args.N) return;
  if (OUT == OK_PARTIAL) {
    float* ws = reinterpret_cast<float*>(args.d);
    ws[((long)blockIdx.z * args.M + row) * args.N + col] = v;
    return;
  }
  if (OUT == OK_WGRAD_OIHW && args.dbias && col == args.wg_c * args.wg_rs) {
    reinterpret_cast<S*>(args.dbias)[row] = Elem<T>::from_f32(v);
    return;
  }
  if (args.bias_mode == 1) v += Elem<T>::to_f32(reinterpret_cast<const S*>(args.bias)[row]);
  else if (args.bias_mode == 2) v += Elem<T>::to_f32(reinterpret_cast<const S*>(args.bias)[col]);
  S* d = reinterpret_cast<S*>(args.d);
  const long idx = out_index<T, OUT>(args, row, col);
  if (args.act == 1) v = fmaxf(v, 0.f);
  else if (args.act == 2 && !keep) v = 0.f;
  d[idx] = Elem<T>::from_f32(v);
}

// ---------------------------------------------------------------- the kernel
template <typename T, int AK, int BKIND, int OUT, int BM, int BN, int BK>
__global__ __launch_bounds__(256) void igemm_kernel(IgemmArgs args_in) {
  IgemmArgs args = args_in;
  if (args.nphase > 1) {
    const PhaseArg& f = args_in.ph[blockIdx.y];
    args.a.p = f.a;
    args.g.ph = f.offa;
    args.g.pw = f.offb;
    args.sub_a = f.sub_a;
    args.sub_b = f.sub_b;
  }
  using S = typename Elem<T>::storage;
  // fp32 tiles of at least 64 x 64 use the 32 x 32 fp32 MFMA: its fragment
  // (32 rows of one k per half-wave) is conflict-free with a row pitch of
  // BK + 2 floats (32 rows land on the 32 even banks, k + 1 on the odd ones);
  // the 16-byte units are then stored as two 8-byte halves
  constexpr bool F32_32 = std::is_same<T, float>::value && BM >= 64 && BN >= 64;
  using MM = std::conditional_t<F32_32, MmaF32x32, Mma<T>>;
  constexpr int VEC = Elem<T>::vec;
  constexpr int PADK = F32_32 ? 2 : VEC;  // row pitch (BK + PADK) elements
  constexpr int LDK = BK + PADK;
  constexpr int KU = BK / VEC;         // units per row per K step
  constexpr int UA = BM * KU / 256;    // units per thread, A
  constexpr int UB = BN * KU / 256;    // units per thread, B
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int FM = WM / MM::TM, FN = WN / MM::TN;
  static_assert(UA >= 1 && UB >= 1 && (BM * KU) % 256 == 0 && (BN * KU) % 256 == 0, "tile");

  __shared__ __attribute__((aligned(16))) S smem[2 * (BM + BN) * LDK];
  S* As = smem;
  S* Bs = smem + 2 * BM * LDK;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave >> 1) * WM, wn = (wave & 1) * WN;

  // XCD-aware tile order: consecutive logical tiles land on one XCD (the
  // hardware deals workgroups round-robin over 8 XCDs), column-major groups of 8
  // row tiles so a group shares its B panel in that XCD's L2.
  const int tiles_m = (args.M + BM - 1) / BM, tiles_n = (args.N + BN - 1) / BN;
  const int nt = tiles_m * tiles_n;
  int pid = blockIdx.x;
  if ((nt & 7) == 0) pid = (pid & 7) * (nt >> 3) + (pid >> 3);
  const int group = 8;
  const int gsz = group * tiles_n;
  const int gid = pid / gsz, first_m = gid * group;
  const int gm = min(tiles_m - first_m, group);
  const int tm = first_m + (pid % gsz) % gm, tn = (pid % gsz) / gm;
  const int m0 = tm * BM, n0 = tn * BN;

  const int kb = blockIdx.z * args.k_chunk;
  const int ke = min(args.K, kb + args.k_chunk);
  const int nk = (ke - kb + BK - 1) / BK;

  Loader<T, AK> la[UA];
  Loader<T, BKIND> lb[UB];
  int a_k[UA], a_r[UA], b_k[UB], b_r[UB];
#pragma unroll
  for (int u = 0; u < UA; ++u) {
    int id = tid + u * 256;
    a_r[u] = Loader<T, AK>::kFastest ? id / KU : id % BM;
    a_k[u] = Loader<T, AK>::kFastest ? (id % KU) * VEC : (id / BM) * VEC;
    la[u].init(args.a, args.g, m0 + a_r[u]);
  }
#pragma unroll
  for (int u = 0; u < UB; ++u) {
    int id = tid + u * 256;
    b_r[u] = Loader<T, BKIND>::kFastest ? id / KU : id % BN;
    b_k[u] = Loader<T, BKIND>::kFastest ? (id % KU) * VEC : (id / BN) * VEC;
    lb[u].init(args.b, args.g, n0 + b_r[u]);
  }

  // fp32: two register sets, the loads of stage k+3 issued after the MFMAs of
  // stage k (every load has two stages of MFMAs to arrive); bf16 uses set 0 only
  S ra[2][UA][VEC], rb[2][UB][VEC];
  auto gload = [&](auto SET, int k0) {
    constexpr int s = decltype(SET)::value;
#pragma unroll
    for (int u = 0; u < UA; ++u) la[u].load(args.a, args.g, k0 + a_k[u], ke, ra[s][u]);
#pragma unroll
    for (int u = 0; u < UB; ++u) lb[u].load(args.b, args.g, k0 + b_k[u], ke, rb[s][u]);
  };
  auto st16 = [&](S* dst, const S* src) {
    if constexpr (F32_32) {
      reinterpret_cast<uint2*>(dst)[0] = reinterpret_cast<const uint2*>(src)[0];
      reinterpret_cast<uint2*>(dst)[1] = reinterpret_cast<const uint2*>(src)[1];
    } else {
      *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
    }
  };
  auto sstore = [&](auto SET, int buf) {
    constexpr int s = decltype(SET)::value;
    S* a = As + buf * BM * LDK;
    S* b = Bs + buf * BN * LDK;
#pragma unroll
    for (int u = 0; u < UA; ++u) st16(a + a_r[u] * LDK + a_k[u], ra[s][u]);
#pragma unroll
    for (int u = 0; u < UB; ++u) st16(b + b_r[u] * LDK + b_k[u], rb[s][u]);
  };

  typename MM::acc_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < MM::NACC; ++v) acc[i][j][v] = 0.f;

  const int fr = MM::frag_row(lane), fk = MM::frag_k(lane);
  auto compute = [&](int buf) {
    const S* a = As + buf * BM * LDK;
    const S* b = Bs + buf * BN * LDK;
#pragma unroll
    for (int kk = 0; kk < BK; kk += MM::TK) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = MM::mma(a + (wm + i * MM::TM + fr) * LDK + kk + fk,
                              b + (wn + j * MM::TN + fr) * LDK + kk + fk, acc[i][j]);
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  if constexpr (std::is_same<T, float>::value) {
    // fp32: register set s holds stages s, s+2, ...; LDS buffer k & 1 holds
    // stage k.  Loads past the block's K range read zeros (never multiplied).
    if (nk > 0) {
      gload(I0{}, kb);
      gload(I1{}, kb + BK);
      sstore(I0{}, 0);
      gload(I0{}, kb + 2 * BK);
    }
    __syncthreads();
    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {
      compute(0);
      sstore(I1{}, 1);
      gload(I1{}, kb + (kt + 3) * BK);
      __syncthreads();
      compute(1);
      if (kt + 2 < nk) {
        sstore(I0{}, 0);
        gload(I0{}, kb + (kt + 4) * BK);
      }
      __syncthreads();
    }
    if (kt < nk) compute(0);  // odd stage count: the last stage is in buffer 0
  } else {
    // bf16 (16-bit elements take a register each): one register set, the loads
    // of stage k+1 in flight during the MFMAs of stage k
    if (nk > 0) {
      gload(I0{}, kb);
      sstore(I0{}, 0);
    }
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int buf = kt & 1;
      if (kt + 1 < nk) gload(I0{}, kb + (kt + 1) * BK);
      compute(buf);
      if (kt + 1 < nk) sstore(I0{}, buf ^ 1);
      __syncthreads();
    }
  }

  // the act-2 mask values are read before the first store (a load may not pass
  // a store to possibly the same memory, so interleaving would serialise them)
  bool keep[FM][FN][MM::NACC];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < MM::NACC; ++v)
        keep[i][j][v] = OUT != OK_PARTIAL && args.act == 2 &&
                        mask_keep<T, OUT>(args, m0 + wm + i * MM::TM + MM::acc_row(lane, v),
                                          n0 + wn + j * MM::TN + MM::acc_col(lane));
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < MM::NACC; ++v)
        store_out<T, OUT>(args, m0 + wm + i * MM::TM + MM::acc_row(lane, v),
                          n0 + wn + j * MM::TN + MM::acc_col(lane), acc[i][j][v], keep[i][j][v]);
}

// Split-K reduction: out(row, col) = sum_z ws[z][row][col] (+ bias), stored by
// OUT; fixed summation order (reduce_splits_block).
template <typename T, int OUT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(IgemmArgs args, const float* ws, int splits) {
  const long total = (long)args.M * args.N;
  reduce_splits_block(ws, splits, total, [&](long i, float s) {
    const int row = (int)(i / args.N), col = (int)(i % args.N);
    store_out<T, OUT>(args, row, col, s, args.act == 2 && mask_keep<T, OUT>(args, row, col));
  });
}

// The same for the weight-gradient scatter (OK_WGRAD_OIHW, no bias or
// activation): block (o, 64-channel chunk) sums the partials of its 64 c x R*S
// columns (rows of the [RS][C] column order, contiguous in c) in split order
// into LDS, then writes dW[o][c0 .. c0+63][0 .. RS) as one contiguous run.
template <typename T>
__global__ __launch_bounds__(256) void splitk_reduce_oihw_kernel(IgemmArgs args, const float* __restrict__ ws,
                                                                 int splits) {
  using S = typename Elem<T>::storage;
  extern __shared__ float tile[];  // [RS][65]
  const int o = blockIdx.x, c0 = blockIdx.y * 64;
  const int C = args.wg_c, RS = args.wg_rs;
  const int nc = min(64, C - c0);
  const long MN = (long)args.M * args.N;
  for (int i = threadIdx.x; i < RS * 64; i += 256) {
    const int rs = i >> 6, cl = i & 63;
    float s = 0.f;
    if (cl < nc) {
      const float* p = ws + (long)o * args.N + (long)rs * C + c0 + cl;
#pragma unroll 8
      for (int z = 0; z < splits; ++z) s += p[z * MN];
    }
    tile[rs * 65 + cl] = s;
  }
  __syncthreads();
  S* d = reinterpret_cast<S*>(args.d) + ((long)o * C + c0) * RS;
  for (int i = threadIdx.x; i < nc * RS; i += 256) {
    const int cl = i / RS, rs = i - cl * RS;
    d[i] = Elem<T>::from_f32(tile[rs * 65 + cl]);
  }
  // the bias column (a B row of ones): the same split order
  if (args.dbias && blockIdx.y == 0 && threadIdx.x == 0) {
    const float* p = ws + (long)o * args.N + (long)RS * C;
    float s = 0.f;
    for (int z = 0; z < splits; ++z) s += p[z * MN];
    reinterpret_cast<S*>(args.dbias)[o] = Elem<T>::from_f32(s);
  }
}

}  // namespace vh
