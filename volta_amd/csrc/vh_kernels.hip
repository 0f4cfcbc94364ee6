// vh_kernels.hip -- kernels other than the MFMA implicit GEMM, plus the typed
// launch helpers the C ABI layer calls.  gfx950 only.
#include "vh_kernels.hpp"

#include <algorithm>
#include <cmath>

namespace vh {

static inline int grid_for(long n, int per_block = 256, int cap = 65535 * 8) {
  long g = (n + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (int)g;
}

// ============================================================== direct conv
// Volta's direct_conv.wgsl:27-105 assigns one output element per invocation; so
// does this kernel (consecutive lanes take consecutive ow, so x loads and y
// stores coalesce).  The f32 sum runs in the reference's CPU order
// ic -> kh -> kw (conv.rs:1370-1407) with separate multiply and add roundings
// (Rust never contracts a*b+c), so f32 results equal Volta's CPU Direct loop
// bit for bit.  The bias is added in fp32 before the single output rounding.
template <typename T>
__global__ __launch_bounds__(256) void direct_fwd_kernel(const typename Elem<T>::storage* __restrict__ x,
                                                         const typename Elem<T>::storage* __restrict__ w,
                                                         const typename Elem<T>::storage* __restrict__ bias,
                                                         typename Elem<T>::storage* __restrict__ y,
                                                         ConvGeom g, long total, int act) {
#pragma clang fp contract(off)
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
    int q = (int)(i % g.Q);
    long t = i / g.Q;
    int p = (int)(t % g.P);
    t /= g.P;
    int o = (int)(t % g.O);
    int n = (int)(t / g.O);
    float s = 0.f;
    const auto* xn = x + (long)n * g.C * g.H * g.W;
    const auto* wo = w + (long)o * g.C * g.R * g.S;
    for (int c = 0; c < g.C; ++c)
      for (int r = 0; r < g.R; ++r) {
        int h = p * g.sh + r - g.ph;
        if (h < 0 || h >= g.H) continue;
        for (int k = 0; k < g.S; ++k) {
          int ww = q * g.sw + k - g.pw;
          if (ww < 0 || ww >= g.W) continue;
          float prod = Elem<T>::to_f32(xn[((long)c * g.H + h) * g.W + ww]) *
                       Elem<T>::to_f32(wo[(c * g.R + r) * g.S + k]);
          s += prod;
        }
      }
    if (bias) s += Elem<T>::to_f32(bias[o]);
    auto v = Elem<T>::from_f32(s);
    // act 1: ReLU of the rounded value (zero unless it is positive)
    if (act == 1 && !(Elem<T>::to_f32(v) > 0.f)) v = Elem<T>::from_f32(0.f);
    y[i] = v;
  }
}

// Direct forward for a few products per output (C*R*S <= 128, R x S of 1x1, 3x3
// or 5x5: a first layer on 1-4 channels).  Block (image n, OB output channels,
// chunk of 256 output positions): one position per lane, whose C*R*S input taps are
// read once and multiplied with the OB channels' weights (staged in LDS as
// fp32), so x is read once per OB outputs instead of once per output, and the
// index math is 32-bit.  Every output is summed exactly as direct_fwd_kernel
// sums it (c -> r -> s, out-of-range taps skipped, separate multiply and add,
// bias in fp32 before the one rounding, ReLU of the rounded value): the
// results are bit-identical, i.e. equal to Volta's CPU Direct loop in f32.
template <typename T, int R, int S, int OB>
__global__ __launch_bounds__(256) void direct_fwd_small_kernel(const typename Elem<T>::storage* __restrict__ x,
                                                               const typename Elem<T>::storage* __restrict__ w,
                                                               const typename Elem<T>::storage* __restrict__ bias,
                                                               typename Elem<T>::storage* __restrict__ y,
                                                               ConvGeom g, int act) {
#pragma clang fp contract(off)
  constexpr int RS = R * S;
  __shared__ float wl[OB][128];
  const int n = blockIdx.x, o0 = blockIdx.y * OB;
  const int CRS = g.C * RS;
  for (int i = threadIdx.x; i < OB * CRS; i += 256) {
    const int o = i / CRS, k = i - o * CRS;
    wl[o][k] = o0 + o < g.O ? Elem<T>::to_f32(w[(long)(o0 + o) * CRS + k]) : 0.f;
  }
  float bv[OB];
#pragma unroll
  for (int o = 0; o < OB; ++o) bv[o] = bias && o0 + o < g.O ? Elem<T>::to_f32(bias[o0 + o]) : 0.f;
  __syncthreads();
  const int PQ = g.P * g.Q, HW = g.H * g.W;
  const auto* xn = x + (long)n * g.C * HW;
  auto* yn = y + ((long)n * g.O + o0) * PQ;
  for (int pq = blockIdx.z * 256 + threadIdx.x; pq < PQ; pq += gridDim.z * 256) {
    uint32_t p, q;
    g.fQ.divmod((uint32_t)pq, p, q);
    const int h0 = (int)p * g.sh - g.ph, w0 = (int)q * g.sw - g.pw;
    float sacc[OB];
#pragma unroll
    for (int o = 0; o < OB; ++o) sacc[o] = 0.f;
    for (int c = 0; c < g.C; ++c) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int h = h0 + r;
        if (h < 0 || h >= g.H) continue;
#pragma unroll
        for (int k = 0; k < S; ++k) {
          const int ww = w0 + k;
          if (ww < 0 || ww >= g.W) continue;
          const float xv = Elem<T>::to_f32(xn[c * HW + h * g.W + ww]);
#pragma unroll
          for (int o = 0; o < OB; ++o) {
            const float prod = xv * wl[o][(c * R + r) * S + k];
            sacc[o] += prod;
          }
        }
      }
    }
#pragma unroll
    for (int o = 0; o < OB; ++o) {
      if (o0 + o >= g.O) break;
      float sv = sacc[o];
      if (bias) sv += bv[o];
      auto v = Elem<T>::from_f32(sv);
      if (act == 1 && !(Elem<T>::to_f32(v) > 0.f)) v = Elem<T>::from_f32(0.f);
      yn[(long)o * PQ + pq] = v;
    }
  }
}

// Input gradient, one input element per lane (conv_backward_input.wgsl:26-89).
// Terms are visited in the reference's order oc -> oh -> ow (conv.rs:458-505),
// skipping the output positions whose receptive field misses the element, with
// unfused multiply/add: f32 results equal Volta's CPU loop bit for bit.
template <typename T>
__global__ __launch_bounds__(256) void direct_dgrad_kernel(const typename Elem<T>::storage* __restrict__ dy,
                                                           const typename Elem<T>::storage* __restrict__ w,
                                                           typename Elem<T>::storage* __restrict__ dx,
                                                           ConvGeom g, long total) {
#pragma clang fp contract(off)
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
    int iw = (int)(i % g.W);
    long t = i / g.W;
    int ih = (int)(t % g.H);
    t /= g.H;
    int c = (int)(t % g.C);
    int n = (int)(t / g.C);
    const int th = ih + g.ph, tw = iw + g.pw;
    // first output row/col whose window reaches this element: oh*sh > th - R
    const int oh0 = th - g.R + 1 <= 0 ? 0 : (th - g.R + 1 + g.sh - 1) / g.sh;
    const int ow0 = tw - g.S + 1 <= 0 ? 0 : (tw - g.S + 1 + g.sw - 1) / g.sw;
    float s = 0.f;
    for (int o = 0; o < g.O; ++o) {
      const auto* dyo = dy + (((long)n * g.O + o) * g.P) * g.Q;
      const auto* wo = w + ((long)o * g.C + c) * g.R * g.S;
      for (int oh = oh0; oh < g.P && oh * g.sh <= th; ++oh) {
        const int r = th - oh * g.sh;
        for (int ow = ow0; ow < g.Q && ow * g.sw <= tw; ++ow) {
          const int k = tw - ow * g.sw;
          float prod = Elem<T>::to_f32(dyo[(long)oh * g.Q + ow]) * Elem<T>::to_f32(wo[r * g.S + k]);
          s += prod;
        }
      }
    }
    dx[i] = Elem<T>::from_f32(s);
  }
}

// Input gradient of a convolution with at most 4 input channels (and
// ConvTranspose2d's forward to at most 4 output channels, e.g. a generator's
// last layer to RGB), where an implicit GEMM would spend over 90 % of its MFMA
// tile on rows past C.  One lane per input position (n, h, w) computes all C of
// its outputs: for every tap (r, s) that reaches an output position (the other
// stride phases are skipped) and every output channel o, one dY load and C
// fused multiply-adds with the weights, held in LDS as fp32 [o][r][s][CC].  fp32
// accumulation; bias and the ReLU-backward mask (zero where mask <= 0) in the
// epilogue, one rounding.  Consecutive lanes take consecutive w, so the dY
// loads of a wave cover one or two runs of a row.
template <typename T, int CC>
__global__ __launch_bounds__(256) void dgrad_smallc_kernel(const typename Elem<T>::storage* __restrict__ dy,
                                                           const typename Elem<T>::storage* __restrict__ w,
                                                           const typename Elem<T>::storage* __restrict__ bias,
                                                           const typename Elem<T>::storage* __restrict__ mask,
                                                           typename Elem<T>::storage* __restrict__ dx, ConvGeom g,
                                                           long total) {
  extern __shared__ float wl[];
  const int RS = g.R * g.S;
  for (int i = threadIdx.x; i < g.O * RS * CC; i += 256) {
    const int c = i % CC, ors = i / CC, o = ors / RS, rs = ors - o * RS;
    wl[i] = c < g.C ? Elem<T>::to_f32(w[((long)o * g.C + c) * RS + rs]) : 0.f;
  }
  __syncthreads();
  const long PQ = (long)g.P * g.Q;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
    const int iw = (int)(i % g.W);
    const long t = i / g.W;
    const int ih = (int)(t % g.H), n = (int)(t / g.H);
    float acc[CC];
#pragma unroll
    for (int c = 0; c < CC; ++c) acc[c] = 0.f;
    const int th = ih + g.ph, tw = iw + g.pw;
    const auto* dyn = dy + (long)n * g.O * PQ;
    // taps r = th mod sh, +sh, ... (r <= th): output row p = (th - r) / sh
    for (int r = th % g.sh; r < g.R && r <= th; r += g.sh) {
      const int p = (th - r) / g.sh;
      if (p >= g.P) continue;
      for (int s = tw % g.sw; s < g.S && s <= tw; s += g.sw) {
        const int q = (tw - s) / g.sw;
        if (q >= g.Q) continue;
        const auto* d0 = dyn + (long)p * g.Q + q;
        const float* w0 = wl + (r * g.S + s) * CC;
        int o = 0;
        for (; o + 4 <= g.O; o += 4) {
          float v[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) v[u] = Elem<T>::to_f32(d0[(o + u) * PQ]);
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int c = 0; c < CC; ++c) acc[c] = fmaf(v[u], w0[(o + u) * RS * CC + c], acc[c]);
        }
        for (; o < g.O; ++o) {
          const float v = Elem<T>::to_f32(d0[o * PQ]);
#pragma unroll
          for (int c = 0; c < CC; ++c) acc[c] = fmaf(v, w0[o * RS * CC + c], acc[c]);
        }
      }
    }
#pragma unroll
    for (int c = 0; c < CC; ++c) {
      if (c >= g.C) break;
      const long idx = (((long)n * g.C + c) * g.H + ih) * g.W + iw;
      float val = acc[c] + (bias ? Elem<T>::to_f32(bias[c]) : 0.f);
      if (mask && !(Elem<T>::to_f32(mask[idx]) > 0.f)) val = 0.f;
      dx[idx] = Elem<T>::from_f32(val);
    }
  }
}

// Sum over the 64 lanes of a wave (butterfly, the same order on every lane).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Tap offsets of one axis of a fixed geometry (taps K, stride ST, padding PD)
// seen from cells: a cell t covers input positions ST*t + e, e < ST.  Position
// e reaches taps k = a(e) + ST*j, j < nj(e), and reads output index
// t + base(e) - j there; dmin..dmax is the span of those offsets over the cell.
template <int K, int ST, int PD> struct CellAxis {
  static constexpr int a(int e) { return (e + PD) % ST; }
  static constexpr int base(int e) { return (e + PD) / ST; }
  static constexpr int nj(int e) { return a(e) < K ? (K - a(e) + ST - 1) / ST : 0; }
  static constexpr int dmin() {
    int m = 1 << 20;
    for (int e = 0; e < ST; ++e)
      if (nj(e) && base(e) - nj(e) + 1 < m) m = base(e) - nj(e) + 1;
    return m;
  }
  static constexpr int dmax() {
    int m = -(1 << 20);
    for (int e = 0; e < ST; ++e)
      if (nj(e) && base(e) > m) m = base(e);
    return m;
  }
};

// dY loads of the cell kernel: buffer loads, so an offset of kCellOOR (past
// any tensor the launch accepts) reads zeros without a branch.
constexpr uint32_t kCellOOR = 0x80000000u;
template <typename T> struct CellLoad;
template <> struct CellLoad<float> {
  static __device__ inline void four(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, float* v) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 u = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0));
    v[0] = u.x, v[1] = u.y, v[2] = u.z, v[3] = u.w;
  }
  static __device__ inline float one(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0));
  }
};
template <> struct CellLoad<bf16> {
  static __device__ inline void four(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, float* v) {
    typedef unsigned int u2 __attribute__((ext_vector_type(2)));
    const u2 u = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, 0));
    v[0] = __uint_as_float(u.x << 16), v[1] = __uint_as_float(u.x & 0xffff0000u);
    v[2] = __uint_as_float(u.y << 16), v[3] = __uint_as_float(u.y & 0xffff0000u);
  }
  static __device__ inline float one(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    return __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, vo, so, 0) << 16);
  }
};

// Input gradient with at most 4 input channels for one fixed tap geometry
// (R, S, stride and padding known at compile time).  A lane owns one cell row
// and four cell columns of one image, a cell being the SH x SW block of input
// positions that together read dY rows t + dmin..dmax and columns v +
// dmin..dmax of the axis; each dY value it loads (one 4-wide load for the
// cells' own columns, single loads for the rest) feeds every tap of every
// position that reads it.  The four waves of a block own the same cells and
// split the output channels; waves 1-3 hand their sums to wave 0 through LDS,
// which adds bias, applies the ReLU-backward mask and stores.  Weights are
// uniform across the block (scalar loads).  fp32 accumulation, one rounding.
template <typename T, int C, int R, int S, int SH, int SW, int PH, int PW>
__global__ __launch_bounds__(256) void dgrad_cell_kernel(const typename Elem<T>::storage* __restrict__ dy,
                                                         const typename Elem<T>::storage* __restrict__ w,
                                                         const typename Elem<T>::storage* __restrict__ bias,
                                                         const typename Elem<T>::storage* __restrict__ mask,
                                                         typename Elem<T>::storage* __restrict__ dx, ConvGeom g,
                                                         int ncq, int nct, long nlanes) {
  using RA = CellAxis<R, SH, PH>;
  using CA = CellAxis<S, SW, PW>;
  constexpr int R0 = RA::dmin(), NR = RA::dmax() - R0 + 1;
  constexpr int C0 = CA::dmin(), NCOL = 4 + CA::dmax() - C0;
  static_assert(C0 <= 0 && R0 <= 0, "cell offsets must include the cell's own row and column");
  constexpr int NOUT = SH * 4 * SW * C, KW = C * R * S;
  static_assert(std::is_same<T, float>::value || KW % 2 == 0, "bf16 weights are read in pairs");
  __shared__ float red[4][3][SH * SW * C][64];

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const long gl = (long)blockIdx.x * 64 + lane;
  const bool active = gl < nlanes;
  const int vq = (int)(gl % ncq);
  const long rest = gl / ncq;
  const int t = (int)(rest % nct), n = (int)(rest / nct);
  const int v0 = 4 * vq;
  const long PQ = (long)g.P * g.Q;
  const int ow = (g.O + 3) / 4, o_beg = wv * ow, o_end = min(g.O, o_beg + ow);

  float acc[NOUT];
#pragma unroll
  for (int k = 0; k < NOUT; ++k) acc[k] = 0.f;
  // byte offsets of the lane's dY values in channel 0 of its image; channel o
  // adds o * P * Q elements through the scalar offset
  constexpr int ES = sizeof(typename Elem<T>::storage);
  constexpr int NEDGE = NCOL - 4;
  uint32_t off_mid[NR], off_edge[NR][NEDGE > 0 ? NEDGE : 1];
  {
    const long img = (long)(active ? n : 0) * g.O * PQ;
#pragma unroll
    for (int rr = 0; rr < NR; ++rr) {
      const int p = t + R0 + rr;
      const bool rowok = active && p >= 0 && p < g.P;
      const long row = img + (long)p * g.Q;
      off_mid[rr] = rowok && v0 < g.Q ? (uint32_t)((row + v0) * ES) : kCellOOR;
#pragma unroll
      for (int e = 0, cc = 0; cc < NCOL; ++cc) {
        const int dq = C0 + cc;
        if (dq >= 0 && dq < 4) continue;
        const int q = v0 + dq;
        off_edge[rr][e++] = rowok && q >= 0 && q < g.Q ? (uint32_t)((row + q) * ES) : kCellOOR;
      }
    }
  }
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)dy, (short)0, (int)((long)g.N * g.O * PQ * ES), 0x00020000);
  auto load = [&](int o, float (&d)[NR][NCOL]) {
    const uint32_t so = (uint32_t)((long)o * PQ * ES);
#pragma unroll
    for (int rr = 0; rr < NR; ++rr) {
      float m4[4];
      CellLoad<T>::four(rsrc, off_mid[rr], so, m4);
#pragma unroll
      for (int e = 0, cc = 0; cc < NCOL; ++cc) {
        const int dq = C0 + cc;
        if (dq >= 0 && dq < 4) d[rr][cc] = m4[dq];
        else d[rr][cc] = CellLoad<T>::one(rsrc, off_edge[rr][e++], so);
      }
    }
  };

  auto compute = [&](int o, const float (&d)[NR][NCOL]) {
    float wk[KW];
    if constexpr (std::is_same<T, float>::value) {
#pragma unroll
      for (int i = 0; i < KW; ++i) wk[i] = w[(long)o * KW + i];
    } else {
      const uint32_t* w32 = reinterpret_cast<const uint32_t*>(w) + (long)o * (KW / 2);
#pragma unroll
      for (int i = 0; i < KW / 2; ++i) {
        const uint32_t u = w32[i];
        wk[2 * i] = __uint_as_float(u << 16), wk[2 * i + 1] = __uint_as_float(u & 0xffff0000u);
      }
    }
#pragma unroll
    for (int er = 0; er < SH; ++er)
#pragma unroll
      for (int j = 0; j < RA::nj(er); ++j) {
        const int r = RA::a(er) + SH * j, rr = RA::base(er) - j - R0;
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int ec = 0; ec < SW; ++ec)
#pragma unroll
            for (int i = 0; i < CA::nj(ec); ++i) {
              const int s = CA::a(ec) + SW * i, cc = k + CA::base(ec) - i - C0;
#pragma unroll
              for (int c = 0; c < C; ++c)
                acc[((er * 4 + k) * SW + ec) * C + c] =
                    fmaf(d[rr][cc], wk[(c * R + r) * S + s], acc[((er * 4 + k) * SW + ec) * C + c]);
            }
      }
  };

  // two register sets: the loads of channel o + 1 are in flight while o is
  // summed (the last one repeats a channel instead of branching)
  float da[NR][NCOL], db[NR][NCOL];
  int o = o_beg;
  if (o < o_end) load(o, da);
  for (; o + 1 < o_end; o += 2) {
    load(o + 1, db);
    compute(o, da);
    load(min(o + 2, o_end - 1), da);
    compute(o + 1, db);
  }
  if (o < o_end) compute(o, da);

  // wave k finishes cell column k of the lane: the other three waves hand it
  // their sums for that column through LDS
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (k == wv) continue;
    const int slot = wv < k ? wv : wv - 1;
#pragma unroll
    for (int er = 0; er < SH; ++er)
#pragma unroll
      for (int j = 0; j < SW * C; ++j) red[k][slot][er * SW * C + j][lane] = acc[(er * 4 + k) * SW * C + j];
  }
  __syncthreads();
  if (!active) return;
  auto finish = [&](auto kc) {
    constexpr int k = decltype(kc)::value;
    const int iw0 = SW * (v0 + k);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const float bc = bias ? Elem<T>::to_f32(bias[c]) : 0.f;
#pragma unroll
      for (int er = 0; er < SH; ++er) {
        const int ih = SH * t + er;
        if (ih >= g.H) continue;
        const long row = (((long)n * C + c) * g.H + ih) * g.W;
#pragma unroll
        for (int ec = 0; ec < SW; ++ec) {
          const int iw = iw0 + ec, j = (er * SW + ec) * C + c;
          if (iw >= g.W) continue;
          float val = acc[(er * 4 + k) * SW * C + ec * C + c] + red[k][0][j][lane] + red[k][1][j][lane] +
                      red[k][2][j][lane] + bc;
          if (mask && !(Elem<T>::to_f32(mask[row + iw]) > 0.f)) val = 0.f;
          dx[row + iw] = Elem<T>::from_f32(val);
        }
      }
    }
  };
  switch (wv) {
    case 0: finish(std::integral_constant<int, 0>()); break;
    case 1: finish(std::integral_constant<int, 1>()); break;
    case 2: finish(std::integral_constant<int, 2>()); break;
    default: finish(std::integral_constant<int, 3>()); break;
  }
}

// Weight gradient of the same layer shape (4x4 taps, stride 2, padding 1, at
// most 4 input channels, at most 64 output channels), fp32 on
// v_mfma_f32_32x32x2f32: D[o][(c, r, s)] = sum over positions (n, p, q) of
// dY[n][o][p][q] * x[n][c][2p - 1 + r][2q - 1 + s].  A stage is one 32-position
// segment of a dY row: its dY tile [o][q] and the four x rows 2p - 1 .. 2p + 2 of
// every channel (columns -1 .. 64 of the segment, zeros outside the image) go
// to LDS through registers, double-buffered, and each wave multiplies a 32 x 32
// quadrant of the 64 x 64 (o x (c, r, s)) tile over the stage's 32 positions.
// Blocks own ranges of stages and write fp32 partials [block][O][C][4][4]
// followed by the bias sums [block][C] (x rows 2p and 2p + 1 of each stage
// cover every row once); a second kernel adds them in block order.
constexpr int kCwQ = 32;                  // positions per stage
constexpr int kCwAP = kCwQ + 2;           // dY tile pitch (o rows): k and k + 1 on even / odd banks
constexpr int kCwXP = 76;                 // x row pitch: 12 * row mod 64 keeps 12 rows' taps apart
constexpr int kCwXR = 17;                 // 16 x rows (c, r) + a zero row for padded columns

__global__ __launch_bounds__(256) void convt_cell_wgrad_kernel(const float* __restrict__ dy,
                                                              const float* __restrict__ x,
                                                              float* __restrict__ part, ConvGeom g, int nseg,
                                                              int stages, int per_block) {
  __shared__ __attribute__((aligned(16))) float as[2][64 * kCwAP];
  __shared__ __attribute__((aligned(16))) float xs[2][kCwXR * kCwXP];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  const int fr = lane & 31, fk = lane >> 5;
  const int C = g.C, O = g.O, NCOL = C * 16;
  const long PQ = (long)g.P * g.Q, HW = (long)g.H * g.W;
  // this lane's fragment rows: A row m = o, B column n = (c, r, s)
  const int aoff = (wm + fr) * kCwAP + fk;
  const int n = wn + fr;
  const int boff = n < NCOL ? ((n >> 2) * kCwXP + (n & 3) + 3 + 2 * fk) : 16 * kCwXP;
  // zero row (padded columns of B) in both buffers
  for (int i = tid; i < 2 * kCwXP; i += 256) xs[i / kCwXP][16 * kCwXP + i % kCwXP] = 0.f;

  const int s_b = blockIdx.x * per_block, s_e = min(stages, s_b + per_block);
  // stage -> (image, dY row, 32-position segment)
  auto decode = [&](int st, int& img, int& p, int& seg) {
    seg = st % nseg;
    const int t = st / nseg;
    p = t % g.P;
    img = t / g.P;
  };
  float4 ra[2];  // dY: 64 o x 8 float4 per stage, two per thread
  float4 rx[2];  // x: 16 rows x 18 float4 (columns 64 seg - 4 + 4j), at most two per thread
  // bias: sums of the x chunks of rows r = 1, 2 (x rows 2p, 2p + 1) and
  // columns 64 seg .. 64 seg + 63, per slot (a slot's channel is fixed)
  float bsum[2] = {0.f, 0.f};
  auto gload = [&](int st) {
    int img, p, seg;
    decode(st, img, p, seg);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = tid + u * 256, o = i >> 3, q4 = i & 7;
      ra[u] = o < O ? *reinterpret_cast<const float4*>(dy + ((long)img * O + o) * PQ + (long)p * g.Q + seg * kCwQ +
                                                       q4 * 4)
                    : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = tid + u * 256;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (i < C * 4 * 18) {
        const int row = i / 18, j = i - row * 18;  // row = (c, r)
        const int c = row >> 2, r = row & 3;
        const int h = 2 * p - 1 + r, col = seg * 2 * kCwQ - 4 + 4 * j;
        if (h >= 0 && h < g.H && col >= 0 && col < g.W)
          v = *reinterpret_cast<const float4*>(x + ((long)img * C + c) * HW + (long)h * g.W + col);
        if ((r == 1 || r == 2) && j >= 1 && j <= 16) bsum[u] += ((v.x + v.y) + v.z) + v.w;
      }
      rx[u] = v;
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = tid + u * 256, o = i >> 3, q4 = i & 7;
      // pitch 34: two 8-byte halves
      float* d = &as[buf][o * kCwAP + q4 * 4];
      *reinterpret_cast<float2*>(d) = make_float2(ra[u].x, ra[u].y);
      *reinterpret_cast<float2*>(d + 2) = make_float2(ra[u].z, ra[u].w);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = tid + u * 256;
      if (i < C * 4 * 18) {
        const int row = i / 18, j = i - row * 18;
        *reinterpret_cast<float4*>(&xs[buf][row * kCwXP + 4 * j]) = rx[u];
      }
    }
  };
  f32x16 acc = f32x16{};
  auto compute = [&](int buf) {
    const float* a = as[buf] + aoff;
    const float* b = xs[buf] + boff;
#pragma unroll
    for (int kk = 0; kk < kCwQ; kk += 2) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[kk], b[2 * kk], acc, 0, 0, 0);
  };
  if (s_b < s_e) {
    gload(s_b);
    sstore(0);
  }
  __syncthreads();
  for (int st = s_b; st < s_e; ++st) {
    const int buf = (st - s_b) & 1;
    if (st + 1 < s_e) gload(st + 1);
    compute(buf);
    if (st + 1 < s_e) sstore(buf ^ 1);
    __syncthreads();
  }
  // partials: lane holds D[o = wm + row(v)][n]
  const long nw = (long)O * NCOL;
  float* pb = part + (long)blockIdx.x * ((nw + C + 3) & ~3L);  // slabs of whole 16-byte quads
  if (n < NCOL) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int o = wm + (v >> 2) * 8 + fk * 4 + (v & 3);
      if (o < O) pb[(long)o * NCOL + n] = acc[v];
    }
  }
  {
    // per-channel block sums in a fixed order: slot i = tid + 256 u holds
    // channel (i / 18) / 4; wave c adds channel c's 512 slots
    float* red = as[0];  // [4][512], free after the last stage's barrier
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = tid + u * 256, ci = i < C * 72 ? (i / 18) >> 2 : -1;
#pragma unroll
      for (int c = 0; c < 4; ++c) red[c * 512 + i] = c == ci ? bsum[u] : 0.f;
    }
    __syncthreads();
    if (wave < C) {
      float t = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) t += red[wave * 512 + k * 64 + lane];
      t = wave_sum(t);
      if (lane == 0) pb[nw + wave] = t;
    }
  }
}

// out: dW [O][C][4][4] = sum over blocks of the partials (slabs of np floats,
// a multiple of 4), then dB [C]; split groups as in the float4 slab reduction
template <typename T>
__global__ __launch_bounds__(256) void convt_cell_wgrad_reduce_kernel(const float* __restrict__ part, int blocks,
                                                                     long np, long nw, int C, int lg_g,
                                                                     typename Elem<T>::storage* __restrict__ dw,
                                                                     typename Elem<T>::storage* __restrict__ db) {
  reduce_splits_vec4_block(
      part, blocks, np, lg_g,
      [&](long i, float v) {
        if (i < nw) dw[i] = Elem<T>::from_f32(v);
        else if (db && i < nw + C) db[i - nw] = Elem<T>::from_f32(v);
      },
      (int)blockIdx.x, (int)gridDim.x);
}

// y[n][c][hw] += bias[c] over an NCHW tensor (fp32 add, one rounding).
template <typename T>
__global__ __launch_bounds__(256) void channel_bias_add_kernel(typename Elem<T>::storage* __restrict__ y,
                                                               const typename Elem<T>::storage* __restrict__ bias,
                                                               int C, long HW, long total) {
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256)
    y[i] = Elem<T>::from_f32(Elem<T>::to_f32(y[i]) + Elem<T>::to_f32(bias[(i / HW) % C]));
}

// Weight gradient: one workgroup per (weight element, position slice); the 256
// lanes stride over output positions and a wavefront reduction (DPP shuffles)
// plus an LDS step combine them into one fp32 partial per slice.

template <typename T>
__global__ __launch_bounds__(256) void direct_wgrad_kernel(const typename Elem<T>::storage* __restrict__ dy,
                                                           const typename Elem<T>::storage* __restrict__ x,
                                                           float* __restrict__ part, ConvGeom g,
                                                           int slice) {
  const int widx = blockIdx.x;  // (o, c, r, s)
  int k = widx % g.S;
  int t = widx / g.S;
  int r = t % g.R;
  t /= g.R;
  int c = t % g.C;
  int o = t / g.C;
  const long npos = (long)g.N * g.P * g.Q;
  long b = (long)blockIdx.y * slice, e = min(npos, b + slice);
  float s = 0.f;
  for (long i = b + threadIdx.x; i < e; i += 256) {
    int q = (int)(i % g.Q);
    long tt = i / g.Q;
    int p = (int)(tt % g.P);
    int n = (int)(tt / g.P);
    int h = p * g.sh + r - g.ph, w = q * g.sw + k - g.pw;
    if (h < 0 || h >= g.H || w < 0 || w >= g.W) continue;
    s += Elem<T>::to_f32(x[(((long)n * g.C + c) * g.H + h) * g.W + w]) *
         Elem<T>::to_f32(dy[(((long)n * g.O + o) * g.P + p) * g.Q + q]);
  }
  s = wave_sum(s);
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) part[(long)blockIdx.y * gridDim.x + widx] = red[0] + red[1] + red[2] + red[3];
}

// Sum of partials [splits][n] -> out[n] (dtype T), fixed order (four waves
// over interleaved splits, then the wave sums in order).
template <typename T>
__global__ __launch_bounds__(256) void sum_partials_kernel(const float* __restrict__ part, int splits, long n,
                                                           typename Elem<T>::storage* __restrict__ out) {
  reduce_splits_block(part, splits, n, [&](long i, float s) { out[i] = Elem<T>::from_f32(s); });
}

// Weight gradient of the Direct algorithm with all R x S taps per block: block
// (o*C + c, slice) walks its slice of output positions once (32-bit index
// math), reads dY once per position and the R x S x values around it, and
// keeps one accumulator per tap; partials [slice][o][c][r][s].
template <typename T, int R, int S>
__global__ __launch_bounds__(256) void direct_wgrad_taps_kernel(const typename Elem<T>::storage* __restrict__ dy,
                                                                const typename Elem<T>::storage* __restrict__ x,
                                                                float* __restrict__ part, ConvGeom g, int slice,
                                                                float* __restrict__ bpart) {
  const int oc = blockIdx.x;
  const int c = oc % g.C, o = oc / g.C;
  const int npos = g.N * g.P * g.Q;
  const int b = blockIdx.y * slice, e = min(npos, b + slice);
  float acc[R * S];
#pragma unroll
  for (int t = 0; t < R * S; ++t) acc[t] = 0.f;
  float bsum = 0.f;  // the bias partial: dY over the slice (blocks of channel 0)
  for (int i = b + threadIdx.x; i < e; i += 256) {
    uint32_t n, pq, p, q;
    g.fPQ.divmod((uint32_t)i, n, pq);
    g.fQ.divmod(pq, p, q);
    const float gv = Elem<T>::to_f32(dy[(((long)n * g.O + o) * g.P + p) * g.Q + q]);
    bsum += gv;
    const long xb = ((long)n * g.C + c) * g.H * g.W;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int h = (int)p * g.sh + r - g.ph;
      if (h < 0 || h >= g.H) continue;
#pragma unroll
      for (int s2 = 0; s2 < S; ++s2) {
        const int w = (int)q * g.sw + s2 - g.pw;
        if (w >= 0 && w < g.W) acc[r * S + s2] += Elem<T>::to_f32(x[xb + (long)h * g.W + w]) * gv;
      }
    }
  }
  __shared__ float red[4][R * S];
#pragma unroll
  for (int t = 0; t < R * S; ++t) {
    const float v = wave_sum(acc[t]);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6][t] = v;
  }
  __syncthreads();
  for (int t = threadIdx.x; t < R * S; t += 256)
    part[((long)blockIdx.y * gridDim.x + oc) * (R * S) + t] = (red[0][t] + red[1][t]) + (red[2][t] + red[3][t]);
  if (bpart && c == 0) {
    const float v = wave_sum(bsum);
    __shared__ float bred[4];
    if ((threadIdx.x & 63) == 0) bred[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) bpart[(long)blockIdx.y * g.O + o] = (bred[0] + bred[1]) + (bred[2] + bred[3]);
  }
}

// Weight (and bias) gradient of the Direct algorithm for 1x1 and 3x3 windows,
// OB output channels per block: block (o-group, input channel c, slice of IT*256 output positions) reads
// each position's OB dY values and its R x S x values once and keeps OB x R*S
// accumulators (+ OB bias sums in the blocks of c = 0) per lane, i.e. x is read
// once per OB output channels.  The lanes' sums are combined through LDS in a
// fixed order (wave, then lane) into one partial per slice: [slice][o][c][r][s]
// and [slice][o], reduced by direct_wgrad_reduce_kernel.
template <typename T, int R, int S, int OB, int IT>
__global__ __launch_bounds__(256) void direct_wgrad_ob_kernel(const typename Elem<T>::storage* __restrict__ dy,
                                                              const typename Elem<T>::storage* __restrict__ x,
                                                              float* __restrict__ part, ConvGeom g,
                                                              float* __restrict__ bpart) {
  constexpr int RS = R * S, NV = OB * RS + OB;  // accumulators per lane
  // rows of 64 lanes at a pitch of 68 floats: the 16-byte row reads of
  // neighbouring threads start on different banks
  constexpr int RP = 68;
  __shared__ float red[4][NV][RP];
  const int o0 = blockIdx.x * OB, c = blockIdx.y, slice = blockIdx.z;
  const int npos = g.N * g.P * g.Q, HW = g.H * g.W, PQ = g.P * g.Q;
  float acc[OB][RS], bs[OB];
#pragma unroll
  for (int o = 0; o < OB; ++o) {
    bs[o] = 0.f;
#pragma unroll
    for (int t = 0; t < RS; ++t) acc[o][t] = 0.f;
  }
  float gv[IT][OB], xv[IT][RS];
  // every load of the lane's IT positions first (out-of-range ones read a
  // clamped address and are zeroed), then the products
#pragma unroll
  for (int u = 0; u < IT; ++u) {
    const int i = (slice * IT + u) * 256 + threadIdx.x;
    const bool ok = i < npos;
    uint32_t n, pq, p, q;
    g.fPQ.divmod((uint32_t)(ok ? i : 0), n, pq);
    g.fQ.divmod(pq, p, q);
    const long db_ = ((long)n * g.O + o0) * PQ + pq;
#pragma unroll
    for (int o = 0; o < OB; ++o) {
      const bool oo = ok && o0 + o < g.O;
      const float v = Elem<T>::to_f32(dy[oo ? db_ + (long)o * PQ : 0]);
      gv[u][o] = oo ? v : 0.f;
    }
    const long xb = ((long)n * g.C + c) * HW;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int h = (int)p * g.sh + r - g.ph;
#pragma unroll
      for (int k = 0; k < S; ++k) {
        const int w = (int)q * g.sw + k - g.pw;
        const bool in = ok && h >= 0 && h < g.H && w >= 0 && w < g.W;
        const float v = Elem<T>::to_f32(x[in ? xb + h * g.W + w : 0]);
        xv[u][r * S + k] = in ? v : 0.f;
      }
    }
  }
#pragma unroll
  for (int u = 0; u < IT; ++u)
#pragma unroll
    for (int o = 0; o < OB; ++o) {
      bs[o] += gv[u][o];
#pragma unroll
      for (int t = 0; t < RS; ++t) acc[o][t] += xv[u][t] * gv[u][o];
    }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 0; o < OB; ++o) {
#pragma unroll
    for (int t = 0; t < RS; ++t) red[wave][o * RS + t][lane] = acc[o][t];
    red[wave][OB * RS + o][lane] = bs[o];
  }
  __syncthreads();
  // each wave's 64 lanes per value (all threads), then the four waves in order
  __shared__ float red2[4][NV];
  for (int idx = threadIdx.x; idx < 4 * NV; idx += 256) {
    const int wv = idx / NV, v = idx - wv * NV;
    const float4* row = reinterpret_cast<const float4*>(red[wv][v]);
    float sum = 0.f;
#pragma unroll
    for (int l4 = 0; l4 < 16; ++l4) {
      const float4 f = row[l4];
      sum += ((f.x + f.y) + (f.z + f.w));
    }
    red2[wv][v] = sum;
  }
  __syncthreads();
  for (int v = threadIdx.x; v < NV; v += 256) {
    const float sum = ((red2[0][v] + red2[1][v]) + red2[2][v]) + red2[3][v];
    if (v < OB * RS) {
      const int o = v / RS, t = v - o * RS;
      if (o0 + o < g.O) part[(long)slice * g.O * g.C * RS + ((long)(o0 + o) * g.C + c) * RS + t] = sum;
    } else if (bpart && c == 0) {
      const int o = v - OB * RS;
      if (o0 + o < g.O) bpart[(long)slice * g.O + o0 + o] = sum;
    }
  }
}

// dW = sum of the slices' partials [slice][nw], and (db non-null) dB = sum of
// the bias partials [slice][O] that follow them; fixed split order.
template <typename T>
__global__ __launch_bounds__(256) void direct_wgrad_reduce_kernel(const float* __restrict__ part, int slices, long nw,
                                                                  int O, typename Elem<T>::storage* __restrict__ dw,
                                                                  typename Elem<T>::storage* __restrict__ db,
                                                                  int nbw) {
  if ((int)blockIdx.x < nbw)
    reduce_splits_block(part, slices, nw, [&](long i, float v) { dw[i] = Elem<T>::from_f32(v); }, (int)blockIdx.x,
                        nbw);
  else
    reduce_splits_block(part + (long)slices * nw, slices, (long)O,
                        [&](long i, float v) { db[i] = Elem<T>::from_f32(v); }, (int)blockIdx.x - nbw,
                        (int)gridDim.x - nbw);
}

static bool direct_wgrad_taps_ok(const ConvGeom& g) {
  const bool shape = (g.R == 3 && g.S == 3) || (g.R == 5 && g.S == 5) || (g.R == 1 && g.S == 1);
  return shape && (long)g.N * g.P * g.Q < (1L << 31) && (long)g.O * g.C <= 65535 * 64;
}

static int direct_wgrad_taps_slices(const ConvGeom& g) {
  const long npos = (long)g.N * g.P * g.Q, oc = (long)g.O * g.C;
  return (int)std::max<long>(1, std::min<long>({(1024 + oc - 1) / oc, (npos + 255) / 256, 1024}));
}

// ============================================================== pad / im2col / col2im// ============================================================== pad / im2col / col2im
template <typename T>
__global__ __launch_bounds__(256) void pad_kernel(const typename Elem<T>::storage* __restrict__ x,
                                                  typename Elem<T>::storage* __restrict__ xp, int BC, int H,
                                                  int W, int ph, int pw, long total) {
  int HP = H + 2 * ph, WP = W + 2 * pw;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
    int wq = (int)(i % WP);
    long t = i / WP;
    int hq = (int)(t % HP);
    long bc = t / HP;
    int h = hq - ph, w = wq - pw;
    typename Elem<T>::storage v = 0;
    if (h >= 0 && h < H && w >= 0 && w < W) v = x[(bc * H + h) * W + w];
    xp[i] = v;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void crop_kernel(const typename Elem<T>::storage* __restrict__ xp,
                                                   typename Elem<T>::storage* __restrict__ x, int H, int W,
                                                   int ph, int pw, long total) {
  int HP = H + 2 * ph, WP = W + 2 * pw;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
    int w = (int)(i % W);
    long t = i / W;
    int h = (int)(t % H);
    long bc = t / H;
    x[i] = xp[(bc * HP + h + ph) * WP + w + pw];
  }
}

// col[(b*HO+oh)*WO+ow][(c*KH+kh)*KW+kw] = x[b][c][oh*sh+kh][ow*sw+kw]  (input pre-padded)
// Lanes walk the column index fastest, so col stores are coalesced.
template <typename T>
__global__ __launch_bounds__(256) void im2col_kernel(const typename Elem<T>::storage* __restrict__ x,
                                                     typename Elem<T>::storage* __restrict__ col, int C, int H,
                                                     int W, int KH, int KW, int SH, int SW, int HO, int WO,
                                                     long total) {
  const int cols = C * KH * KW;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
    int cc = (int)(i % cols);
    long row = i / cols;
    int kw = cc % KW;
    int t = cc / KW;
    int kh = t % KH;
    int c = t / KH;
    int ow = (int)(row % WO);
    long t2 = row / WO;
    int oh = (int)(t2 % HO);
    long b = t2 / HO;
    col[i] = x[((b * C + c) * H + oh * SH + kh) * W + ow * SW + kw];
  }
}

// Gather form of col2im (no atomics): each input element sums every column
// entry that im2col copied it into.  fp32 accumulation.
template <typename T>
__global__ __launch_bounds__(256) void col2im_kernel(const typename Elem<T>::storage* __restrict__ col,
                                                     typename Elem<T>::storage* __restrict__ x, int C, int H,
                                                     int W, int KH, int KW, int SH, int SW, int HO, int WO,
                                                     long total) {
  const int cols = C * KH * KW;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
    int w = (int)(i % W);
    long t = i / W;
    int h = (int)(t % H);
    t /= H;
    int c = (int)(t % C);
    long b = t / C;
    float s = 0.f;
    for (int kh = 0; kh < KH; ++kh) {
      int a = h - kh;
      if (a < 0 || a % SH) continue;
      int oh = a / SH;
      if (oh >= HO) continue;
      for (int kw = 0; kw < KW; ++kw) {
        int bb = w - kw;
        if (bb < 0 || bb % SW) continue;
        int ow = bb / SW;
        if (ow >= WO) continue;
        s += Elem<T>::to_f32(col[((b * HO + oh) * WO + ow) * cols + (c * KH + kh) * KW + kw]);
      }
    }
    x[i] = Elem<T>::from_f32(s);
  }
}

// Input gradient of the Im2col path straight from the fp32 column gradient
// stored transposed, dcolT[(c*KH+kh)*KW+kw][(b*HO+oh)*WO+ow] (the GEMM's own
// output layout, so it is never rounded to bf16), cropping the padding:
// x[b][c][h][w] sums the entries whose padded position (h+ph, w+pw) they copy.
template <typename T>
__global__ __launch_bounds__(256) void col2im_t_kernel(const float* __restrict__ dcolT,
                                                       typename Elem<T>::storage* __restrict__ x, int C, int H,
                                                       int W, int KH, int KW, int SH, int SW, int PH, int PW,
                                                       int HO, int WO, long M, long total) {
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
    int w = (int)(i % W);
    long t = i / W;
    int h = (int)(t % H);
    t /= H;
    int c = (int)(t % C);
    long b = t / C;
    const int hp = h + PH, wp = w + PW;
    float s = 0.f;
    for (int kh = 0; kh < KH; ++kh) {
      int a = hp - kh;
      if (a < 0 || a % SH) continue;
      int oh = a / SH;
      if (oh >= HO) continue;
      for (int kw = 0; kw < KW; ++kw) {
        int bb = wp - kw;
        if (bb < 0 || bb % SW) continue;
        int ow = bb / SW;
        if (ow >= WO) continue;
        s += dcolT[(long)((c * KH + kh) * KW + kw) * M + (b * HO + oh) * WO + ow];
      }
    }
    x[i] = Elem<T>::from_f32(s);
  }
}

// ============================================================== weight re-layouts
// src viewed as [A][B][RS]; dst[a][rs'][b] (swap = 0) or dst[b][rs'][a] (swap = 1)
// with rs' = rs, or rs' = RS-1-rs (flip = 1: the 180-degree kernel rotation that
// turns a stride-1 input gradient into a forward convolution).
//
// Both are batched transposes through an LDS tile: batch t holds a source
// matrix [R1][R2] and dst[t][j][i] = src[t][i][colmap(j)], where colmap keeps
// groups of RS columns together and flips inside a group.  swap = 0: batch a,
// R1 = B, R2 = RS; swap = 1: one batch, R1 = A, R2 = B*RS.  Loads walk source
// rows, stores walk destination rows (both coalesced); a tile holds whole
// column groups (TJ <= 64 is a multiple of RS), so colmap never leaves the tile.
template <int TI, typename T>
__global__ __launch_bounds__(256) void relayout_kernel(const typename Elem<T>::storage* __restrict__ src,
                                                       typename Elem<T>::storage* __restrict__ dst, int R1, int R2,
                                                       int RS, int flip, int TJ) {
  using S = typename Elem<T>::storage;
  __shared__ S tile[TI][65];
  const size_t bofs = (size_t)blockIdx.z * R1 * R2;
  const int j0 = blockIdx.x * TJ, i0 = blockIdx.y * TI;
  // every thread issues all of its loads before the first LDS store
  constexpr int NE = TI * 64 / 256;
  S v[NE];
#pragma unroll
  for (int k = 0; k < NE; ++k) {
    const int e = threadIdx.x + k * 256;
    const int i = e / TJ, jj = e - i * TJ;
    v[k] = (e < TI * TJ && i0 + i < R1 && j0 + jj < R2) ? src[bofs + (size_t)(i0 + i) * R2 + j0 + jj] : S{};
  }
#pragma unroll
  for (int k = 0; k < NE; ++k) {
    const int e = threadIdx.x + k * 256;
    const int i = e / TJ, jj = e - i * TJ;
    if (e < TI * TJ) tile[i][jj] = v[k];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < TI * TJ; e += 256) {
    const int jj = e / TI, i = e - jj * TI;
    const int j = j0 + jj;
    if (i0 + i < R1 && j < R2) {
      const int g = jj / RS, r = jj - g * RS;
      dst[bofs + (size_t)j * R1 + i0 + i] = tile[i][g * RS + (flip ? RS - 1 - r : r)];
    }
  }
}

// Grouped weight layout of the bf16 stride-1 kernel (vh_halo.hip): for a
// GEMM with M rows (output channels of the convolution the kernel computes) and
// contraction channels K (multiple of 16), dst[kg][m][unit][8] holds, in units
// 2*tap and 2*tap+1, channels 16*kg + 0..7 and 16*kg + 8..15 of tap `tap`, and
// zeros in the last unit (2*RS): each row m is 2*RS+1 16-byte units, the pitch
// the kernel's LDS copy of a weight tile uses, so the tile of one 16-channel
// group and a range of rows is one contiguous run that lands in LDS unchanged.
// mode 0: M = O, K = C, from W[m][k][tap] (forward); mode 1: M = C, K = O, from
// W[k][m][tap] with the taps rotated 180 degrees (input gradient as a forward
// convolution).  One thread per 16-byte unit of dst: its eight elements are
// eight independent gathers (all in flight at once -- the pass is a single
// memory round trip, latency-bound) and one 16-byte store.
__global__ __launch_bounds__(256) void relayout_grouped_kernel(const uint16_t* __restrict__ src,
                                                               uint16_t* __restrict__ dst, int M, int K, int RS,
                                                               int mode, FastDiv fU, FastDiv fM) {
  // K is padded to whole groups of 16; the padding channels are zero
  const uint32_t U = 2u * (uint32_t)RS + 1u;  // units per row
  const uint32_t units = (uint32_t)M * (uint32_t)((K + 15) / 16) * U;
  for (uint32_t d = blockIdx.x * 256u + threadIdx.x; d < units; d += gridDim.x * 256u) {
    uint32_t t2, unit, kg, m;
    fU.divmod(d, t2, unit);
    fM.divmod(t2, kg, m);
    const uint32_t tap = unit >> 1, k0 = kg * 16u + (unit & 1u) * 8u;
    // element i: channel k0 + i (src stride RS along k for mode 0, M * RS for mode 1)
    const uint32_t base = mode == 0 ? (m * (uint32_t)K + k0) * RS + tap : (k0 * (uint32_t)M + m) * RS + ((uint32_t)RS - 1u - tap);
    const uint32_t step = mode == 0 ? (uint32_t)RS : (uint32_t)M * RS;
    const bool row_ok = unit + 1u < U;
    uint16_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = row_ok && k0 + i < (uint32_t)K ? src[base + i * step] : (uint16_t)0;
    uint4 o;
    o.x = v[0] | ((uint32_t)v[1] << 16);
    o.y = v[2] | ((uint32_t)v[3] << 16);
    o.z = v[4] | ((uint32_t)v[5] << 16);
    o.w = v[6] | ((uint32_t)v[7] << 16);
    reinterpret_cast<uint4*>(dst)[d] = o;
  }
}

int run_relayout_grouped(const void* w, void* dst, int M, int K, int RS, int mode, hipStream_t st) {
  relayout_grouped_kernel<<<grid_for((long)M * ((K + 15) / 16) * (2 * RS + 1)), 256, 0, st>>>(
      (const uint16_t*)w, (uint16_t*)dst, M, K, RS, mode, FastDiv((uint32_t)(2 * RS + 1)), FastDiv((uint32_t)M));
  VH_LAUNCH_CHECK();
  return VH_OK;
}

// Weights of the stride phases of an input gradient, all phases in one pass:
// phase (a, b) (its first taps kh0 = (a + ph) mod sh, kw0 = (b + pw) mod sw)
// gets dst[c][i][j][o] = w[o][c][kh0 + sh*i][kw0 + sw*j] for the Rc x Sc taps
// that reach its input positions -- the A operand of a stride-1 implicit GEMM.
// Phases are stored one after another (offsets in the table).  Tap (kh, kw)
// belongs to the phase with kh0 = kh mod sh, kw0 = kw mod sw (at most one), so
// the pass walks w once and scatters each element to its phase.
template <typename T>
__global__ __launch_bounds__(256) void relayout_phase_kernel(const typename Elem<T>::storage* __restrict__ w,
                                                             typename Elem<T>::storage* __restrict__ dst, int O,
                                                             int C, int R, int S, int sh, int sw, PhaseTable tab) {
  const long total = (long)O * C * R * S;
  for (long s_ = (long)blockIdx.x * 256 + threadIdx.x; s_ < total; s_ += (long)gridDim.x * 256) {
    const int kw = (int)(s_ % S);
    long t = s_ / S;
    const int kh = (int)(t % R);
    t /= R;
    const int c = (int)(t % C);
    const int o = (int)(t / C);
    for (int pi = 0; pi < tab.n; ++pi) {
      const int kh0 = tab.kh0[pi], kw0 = tab.kw0[pi];
      if (kh % sh != kh0 || kw % sw != kw0) continue;
      const int i = kh / sh, j = kw / sw, Rc = tab.rc[pi], Sc = tab.sc[pi];
      dst[tab.off[pi] + (((long)c * Rc + i) * Sc + j) * O + o] = w[s_];
    }
  }
}

// The same map with one thread per weight row (o, c), o fastest across the
// lanes: a thread reads its R*S contiguous taps, and each tap's stores from a
// wave cover consecutive o of one destination row (coalesced) -- the
// element-wise map above scatters every store to its own cache line.  tap[t]
// (t = kh * S + kw) = phase index | i << 8 | j << 16 of the tap (-1: in no phase).
struct PhaseTaps {
  int tap[64];
};
template <typename T>
__global__ __launch_bounds__(256) void relayout_phase_rows_kernel(const typename Elem<T>::storage* __restrict__ w,
                                                                  typename Elem<T>::storage* __restrict__ dst, int O,
                                                                  int C, int RS, PhaseTable tab, PhaseTaps taps) {
  const long total = (long)O * C;
  for (long d = (long)blockIdx.x * 256 + threadIdx.x; d < total; d += (long)gridDim.x * 256) {
    const int o = (int)(d % O), c = (int)(d / O);
    const typename Elem<T>::storage* src = w + ((long)o * C + c) * RS;
    auto put = [&](int t, typename Elem<T>::storage v) {
      const int m = taps.tap[t], pi = m & 255, i = (m >> 8) & 255, j = m >> 16;
      if (m >= 0) dst[tab.off[pi] + (((long)c * tab.rc[pi] + i) * tab.sc[pi] + j) * O + o] = v;
    };
    if constexpr (std::is_same<T, float>::value) {
      if (RS % 4 == 0) {  // the row as 16-byte loads (w 16-byte aligned: checked by the caller)
        for (int t = 0; t < RS; t += 4) {
          const float4 v = *reinterpret_cast<const float4*>(src + t);
          put(t, v.x);
          put(t + 1, v.y);
          put(t + 2, v.z);
          put(t + 3, v.w);
        }
        continue;
      }
    }
    for (int t = 0; t < RS; ++t) put(t, src[t]);
  }
}

// Element-wise form of the same map for windows of more than 64 taps.
template <typename T>
__global__ __launch_bounds__(256) void relayout_simple_kernel(const typename Elem<T>::storage* __restrict__ src,
                                                              typename Elem<T>::storage* __restrict__ dst, int A,
                                                              int B, int RS, int swap, int flip, FastDiv fRS,
                                                              FastDiv fInner) {
  const uint32_t total = (uint32_t)A * B * RS;
  for (uint32_t d = blockIdx.x * 256u + threadIdx.x; d < total; d += gridDim.x * 256u) {
    uint32_t t, inner, outer, rd;
    fInner.divmod(d, t, inner);  // inner = a (swap) or b
    fRS.divmod(t, outer, rd);    // outer = b (swap) or a
    const uint32_t rs = flip ? (uint32_t)RS - 1u - rd : rd;
    const uint32_t s = swap ? (inner * (uint32_t)B + outer) * RS + rs : (outer * (uint32_t)B + inner) * RS + rs;
    dst[d] = src[s];
  }
}

// ============================================================== reductions
// Per-channel sum of an NCHW tensor [N][C][HW] -> partial[split][C].
template <typename T>
__global__ __launch_bounds__(256) void channel_sum_kernel(const typename Elem<T>::storage* __restrict__ x, int N,
                                                          int C, int HW, float* __restrict__ part, int nslice) {
  const int c = blockIdx.x;
  const long len = (long)N * HW;
  const long per = (len + nslice - 1) / nslice;
  const long b = (long)blockIdx.y * per, e = min(len, b + per);
  float s = 0.f;
  for (long i = b + threadIdx.x; i < e; i += 256) {
    long n = i / HW, hw = i % HW;
    s += Elem<T>::to_f32(x[(n * C + c) * HW + hw]);
  }
  s = wave_sum(s);
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) part[(long)blockIdx.y * C + c] = red[0] + red[1] + red[2] + red[3];
}

typedef unsigned int u32x4w __attribute__((ext_vector_type(4)));

// Sum of the elements of a 16-byte chunk (8 bf16 or 4 f32), in element order.
template <typename T>
__device__ __forceinline__ float vec_sum(const u32x4w v);
template <>
__device__ __forceinline__ float vec_sum<bf16>(const u32x4w v) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s += __uint_as_float(v[i] << 16);
    s += __uint_as_float(v[i] & 0xffff0000u);
  }
  return s;
}
template <>
__device__ __forceinline__ float vec_sum<float>(const u32x4w v) {
  return ((__uint_as_float(v[0]) + __uint_as_float(v[1])) + __uint_as_float(v[2])) + __uint_as_float(v[3]);
}

// Per-channel sum, planes of whole 16-byte chunks (HW a multiple of 16 bytes):
// block (c, n, hs) adds slice hs of plane (n, c) -> partial[n * hsl + hs][C].
template <typename T>
__global__ __launch_bounds__(256) void channel_sum_planes_kernel(const typename Elem<T>::storage* __restrict__ x,
                                                                 int C, int HWv, int hsl,
                                                                 float* __restrict__ part) {
  using S = typename Elem<T>::storage;
  constexpr int VE = 16 / sizeof(S);
  const int c = blockIdx.x, n = blockIdx.y, hs = blockIdx.z;
  const int per = (HWv + hsl - 1) / hsl;
  const int b = hs * per, e = min(HWv, b + per);
  const u32x4w* src = reinterpret_cast<const u32x4w*>(x + ((long)n * C + c) * HWv * VE);
  float s0 = 0.f, s1 = 0.f;
  int k = b + threadIdx.x;
  for (; k + 256 < e; k += 512) {
    const u32x4w v0 = src[k], v1 = src[k + 256];
    s0 += vec_sum<T>(v0);
    s1 += vec_sum<T>(v1);
  }
  if (k < e) s0 += vec_sum<T>(src[k]);
  float s = wave_sum(s0 + s1);
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) part[((long)n * hsl + hs) * C + c] = (red[0] + red[1]) + (red[2] + red[3]);
}

// Column sums of a row-major [M][N] matrix -> partial[split][N]; lanes walk columns.
template <typename T>
__global__ __launch_bounds__(256) void column_sum_kernel(const typename Elem<T>::storage* __restrict__ x, int M,
                                                         int N, float* __restrict__ part, int rows_per) {
  int col = blockIdx.x * 256 + threadIdx.x;
  if (col >= N) return;
  int r0 = blockIdx.y * rows_per, r1 = min(M, r0 + rows_per);
  float s = 0.f;
  for (int r = r0; r < r1; ++r) s += Elem<T>::to_f32(x[(long)r * N + col]);
  part[(long)blockIdx.y * N + col] = s;
}

// Same sums with VE = 16 / sizeof(element) columns per lane (16-byte loads; N %
// VE == 0, 16-byte aligned rows): the rows of a slice are added in the same
// order, so the results equal the one-column kernel's.
template <typename T>
__global__ __launch_bounds__(256) void column_sum_vec_kernel(const typename Elem<T>::storage* __restrict__ x, int M,
                                                             int N, float* __restrict__ part, int rows_per) {
  using S = typename Elem<T>::storage;
  constexpr int VE = 16 / sizeof(S);
  const int col = (blockIdx.x * 256 + threadIdx.x) * VE;
  if (col >= N) return;
  const int r0 = blockIdx.y * rows_per, r1 = min(M, r0 + rows_per);
  float s[VE] = {};
#pragma unroll 8
  for (int r = r0; r < r1; ++r) {
    const uint4 v = *reinterpret_cast<const uint4*>(x + (long)r * N + col);
    const S* e = reinterpret_cast<const S*>(&v);
#pragma unroll
    for (int k = 0; k < VE; ++k) s[k] += Elem<T>::to_f32(e[k]);
  }
  float* o = part + (long)blockIdx.y * N + col;
#pragma unroll
  for (int k = 0; k < VE; k += 4) *reinterpret_cast<float4*>(o + k) = make_float4(s[k], s[k + 1], s[k + 2], s[k + 3]);
}

// Channel sums from column sums of [N][C * HW]: block c adds part[z][c * HW +
// hw] over every slice z and position hw, in a fixed order (four interleaved
// accumulators per lane, then the lanes' butterfly, then the waves in order).
template <typename T>
__global__ __launch_bounds__(256) void channel_segment_sum_kernel(const float* __restrict__ part, int slices, int C,
                                                                  int HW, FastDiv fHW,
                                                                  typename Elem<T>::storage* __restrict__ out) {
  const int c = blockIdx.x, tid = threadIdx.x;
  const long L = (long)C * HW;
  const int tot = slices * HW;
  auto at = [&](int i) {
    uint32_t z, hw;
    fHW.divmod((uint32_t)i, z, hw);
    return part[(long)z * L + (long)c * HW + hw];
  };
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  int i = tid;
  for (; i + 768 < tot; i += 1024) {
    const float v0 = at(i), v1 = at(i + 256), v2 = at(i + 512), v3 = at(i + 768);
    a0 += v0, a1 += v1, a2 += v2, a3 += v3;
  }
  for (; i < tot; i += 256) a0 += at(i);
  const float s = wave_sum((a0 + a1) + (a2 + a3));
  __shared__ float red[4];
  if ((tid & 63) == 0) red[tid >> 6] = s;
  __syncthreads();
  if (tid == 0) out[c] = Elem<T>::from_f32((red[0] + red[1]) + (red[2] + red[3]));
}

// Fixed-order sum of partial slabs part[z][i] (z < splits, i < n, n % 4 == 0,
// 16-byte aligned slabs) read as float4 quads (reduce_splits_vec4_block).
template <typename T>
__global__ __launch_bounds__(256) void sum_partials_vec4_kernel(const float* __restrict__ part, int splits, long n,
                                                                typename Elem<T>::storage* __restrict__ out,
                                                                int lg_g) {
  reduce_splits_vec4_block(part, splits, n, lg_g, [&](long i, float v) { out[i] = Elem<T>::from_f32(v); },
                           (int)blockIdx.x, (int)gridDim.x);
}

// ============================================================== pixel shuffle
// out[b][c][h*r+i][w*r+j] = in[b][c*r*r+i*r+j][h][w]; forward walks the output
// (coalesced stores), backward walks the input gradient.
template <typename T>
__global__ __launch_bounds__(256) void pixel_shuffle_kernel(const typename Elem<T>::storage* __restrict__ in,
                                                            typename Elem<T>::storage* __restrict__ out, int C,
                                                            int H, int W, int r, long total, int backward) {
  const int HO = H * r, WO = W * r;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
    if (!backward) {
      int wo = (int)(i % WO);
      long t = i / WO;
      int ho = (int)(t % HO);
      long bc = t / HO;  // b*C + c
      int h = ho / r, ii = ho - h * r, w = wo / r, jj = wo - w * r;
      out[i] = in[((bc * r + ii) * r + jj) * H * W + (long)h * W + w];
    } else {
      int w = (int)(i % W);
      long t = i / W;
      int h = (int)(t % H);
      t /= H;
      int rr = (int)(t % (r * r));
      long bc = t / (r * r);
      int ii = rr / r, jj = rr - ii * r;
      out[i] = in[(bc * HO + (long)h * r + ii) * WO + (long)w * r + jj];
    }
  }
}

// Vectorised pixel shuffle for r in 2..4 and W a multiple of VE = 16 / sizeof(S):
// work item (b, c, ho, w0) covers VE input columns w0.. of the r input rows that
// output row ho interleaves (channels (c*r + ho%r)*r + j, row ho/r), i.e. VE*r
// contiguous output elements.  Forward reads the r input chunks and writes the
// interleaved run; backward reads the run and writes the r chunks.
template <typename T, int R>
__global__ __launch_bounds__(256) void pixel_shuffle_vec_kernel(const typename Elem<T>::storage* __restrict__ in,
                                                                typename Elem<T>::storage* __restrict__ out,
                                                                int H, int W, int items, int backward) {
  using S = typename Elem<T>::storage;
  constexpr int VE = 16 / sizeof(S);
  const int item = blockIdx.x * 256 + threadIdx.x;
  if (item >= items) return;
  const int wv = W / VE, HO = H * R, WO = W * R;
  const int w0 = (item % wv) * VE;
  const int row = item / wv;  // (b*C + c) * HO + ho
  const int ho = row % HO, bc = row / HO;
  const int h = ho / R, ii = ho - h * R;
  // input-side plane of channel (c*R + ii)*R + j at row h: bc*R*R + ii*R + j
  const long in0 = ((long)(bc * R + ii) * R) * H * W + (long)h * W + w0;
  const long o0 = (long)row * WO + (long)w0 * R;
  S chunk[R][VE];
  S run[R * VE];
  // The runs of a wave's 64 items are one contiguous span of 64 R chunks (rows
  // follow each other in the output).  Forward: a whole wave stores that span
  // with R instructions of 64 consecutive chunks each, exchanging chunks
  // through LDS (chunk u of the span is chunk u % R of item u / R), instead of
  // R instructions whose lanes are R chunks apart (configs[4], r = 3: 22.1 ->
  // 18.3 us).  LDS work of one wave only: a wave barrier after its stores.
  __shared__ u32x4w xs[4][64 * R];
  const int lane = threadIdx.x & 63, wv4 = threadIdx.x >> 6;
  const bool whole = item - lane + 64 <= items;  // wave-uniform
  const long span0 = o0 - (long)lane * R * VE;     // the wave's first output element
  if (!backward) {
#pragma unroll
    for (int j = 0; j < R; ++j)
      *reinterpret_cast<u32x4w*>(chunk[j]) = *reinterpret_cast<const u32x4w*>(in + in0 + (long)j * H * W);
#pragma unroll
    for (int k = 0; k < R * VE; ++k) run[k] = chunk[k % R][k / R];
    if (whole) {
#pragma unroll
      for (int j = 0; j < R; ++j) xs[wv4][R * lane + j] = *reinterpret_cast<const u32x4w*>(run + j * VE);
      // every lane's LDS stores complete before any lane reads another lane's slot
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int j = 0; j < R; ++j)
        *reinterpret_cast<u32x4w*>(out + span0 + (long)(64 * j + lane) * VE) = xs[wv4][64 * j + lane];
      return;
    }
#pragma unroll
    for (int j = 0; j < R; ++j)
      *reinterpret_cast<u32x4w*>(out + o0 + j * VE) = *reinterpret_cast<const u32x4w*>(run + j * VE);
  } else {
    // in = output-shaped gradient, out = input-shaped gradient (loads R chunks
    // apart per lane: measured as fast as the LDS exchange, which is kept for
    // the stores only)
    const long r0 = o0, c0 = in0;
#pragma unroll
    for (int j = 0; j < R; ++j)
      *reinterpret_cast<u32x4w*>(run + j * VE) = *reinterpret_cast<const u32x4w*>(in + r0 + j * VE);
#pragma unroll
    for (int k = 0; k < R * VE; ++k) chunk[k % R][k / R] = run[k];
#pragma unroll
    for (int j = 0; j < R; ++j)
      *reinterpret_cast<u32x4w*>(out + c0 + (long)j * H * W) = *reinterpret_cast<const u32x4w*>(chunk[j]);
  }
}

// ============================================================== glue: ReLU, sum loss
// ReLU: y = x > 0 ? x : +0 (NaN -> 0), backward dx = x > 0 ? g : 0; 16-byte
// vectors when the range allows, one element per lane otherwise.
template <typename T>
__device__ __forceinline__ bool pos(typename Elem<T>::storage v) {
  return Elem<T>::to_f32(v) > 0.f;
}

template <typename T>
__global__ __launch_bounds__(256) void relu_kernel(const typename Elem<T>::storage* __restrict__ x,
                                                   const typename Elem<T>::storage* __restrict__ g,
                                                   typename Elem<T>::storage* __restrict__ y, long n, int vec) {
  using S = typename Elem<T>::storage;
  constexpr int VE = 16 / sizeof(S);
  const long nv = vec ? n / VE : 0;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < nv; i += (long)gridDim.x * 256) {
    S xv[VE], gv[VE], out[VE];
    *reinterpret_cast<uint4*>(xv) = reinterpret_cast<const uint4*>(x)[i];
    if (g) *reinterpret_cast<uint4*>(gv) = reinterpret_cast<const uint4*>(g)[i];
#pragma unroll
    for (int j = 0; j < VE; ++j) out[j] = pos<T>(xv[j]) ? (g ? gv[j] : xv[j]) : S(0);
    reinterpret_cast<uint4*>(y)[i] = *reinterpret_cast<const uint4*>(out);
  }
  for (long i = nv * VE + (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256)
    y[i] = pos<T>(x[i]) ? (g ? g[i] : x[i]) : S(0);
}

// Sum of n elements: block b adds the contiguous slice b (lanes stride the
// slice, then a fixed butterfly and wave order) into part[b]; a second pass
// adds the partials in index order.  When x is 16-byte aligned the slices
// start on 16-byte boundaries and lanes read whole 16-byte chunks.  The
// order depends only on n and that alignment.
template <typename T>
__global__ __launch_bounds__(256) void sum_slices_kernel(const typename Elem<T>::storage* __restrict__ x, long n,
                                                         long per, float* __restrict__ part, int vec) {
  using S = typename Elem<T>::storage;
  constexpr int VE = 16 / sizeof(S);
  const long b = (long)blockIdx.x * per, e = min(n, b + per);
  float s = 0.f;
  long i0 = b;
  if (vec) {  // per is a multiple of VE and x is 16-byte aligned: whole 16-byte chunks first
    const long nv = (e - b) / VE;
    const uint4* xv = reinterpret_cast<const uint4*>(x + b);
    for (long k = threadIdx.x; k < nv; k += 256) {
      S v[VE];
      *reinterpret_cast<uint4*>(v) = xv[k];
      float t = 0.f;
#pragma unroll
      for (int j = 0; j < VE; ++j) t += Elem<T>::to_f32(v[j]);
      s += t;
    }
    i0 = b + nv * VE;
  }
  for (long i = i0 + threadIdx.x; i < e; i += 256) s += Elem<T>::to_f32(x[i]);
  s = wave_sum(s);
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ __launch_bounds__(256) void sum_partials_scalar_kernel(const float* __restrict__ part, int nb,
                                                                  float* __restrict__ out) {
  float s = 0.f;
  for (int i = threadIdx.x; i < nb; i += 256) s += part[i];
  s = wave_sum(s);
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) out[0] = (red[0] + red[1]) + (red[2] + red[3]);
}

// ============================================================== storage: casts and layouts
// dtype conversion: bf16 -> f32 exact, f32 -> bf16 round-to-nearest-even (NaN kept quiet).
template <typename From, typename To>
__global__ __launch_bounds__(256) void cast_kernel(const typename Elem<From>::storage* __restrict__ src,
                                                   typename Elem<To>::storage* __restrict__ dst, long n) {
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256)
    dst[i] = Elem<To>::from_f32(Elem<From>::to_f32(src[i]));
}

// out[b][c][r] = in[b][r][c] for B matrices of R x Cc (NCHW <-> NHWC: R = C, Cc =
// H*W or the reverse); 32 x 32 tiles through LDS, both sides coalesced.
template <typename T>
__global__ __launch_bounds__(256) void batched_transpose_kernel(const typename Elem<T>::storage* __restrict__ in,
                                                                typename Elem<T>::storage* __restrict__ out, int R,
                                                                int Cc) {
  using S = typename Elem<T>::storage;
  __shared__ S t[32][33];
  const long off = (long)blockIdx.z * R * Cc;
  const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
#pragma unroll
  for (int k = 0; k < 32; k += 8) {
    const int r = r0 + ty + k, c = c0 + tx;
    if (r < R && c < Cc) t[ty + k][tx] = in[off + (long)r * Cc + c];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 32; k += 8) {
    const int c = c0 + ty + k, r = r0 + tx;
    if (c < Cc && r < R) out[off + (long)c * R + r] = t[tx][ty + k];
  }
}

// ============================================================== the step after dW
// a += b (gradient accumulation).
template <typename T>
__global__ __launch_bounds__(256) void add_inplace_kernel(typename Elem<T>::storage* __restrict__ a,
                                                          const typename Elem<T>::storage* __restrict__ b, long n) {
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256)
    a[i] = Elem<T>::from_f32(Elem<T>::to_f32(a[i]) + Elem<T>::to_f32(b[i]));
}

// One optimizer update per element, f32, the formulas of the WGSL optimizer
// step in the same order, without contraction into FMAs.
__global__ __launch_bounds__(256) void optimizer_step_kernel(float* __restrict__ param,
                                                             const float* __restrict__ grad, float* __restrict__ s1,
                                                             float* __restrict__ s2, int op, float lr, float beta1,
                                                             float beta2, float mh, float vh, float eps, float wd,
                                                             long n) {
#pragma clang fp contract(off)
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    float g = grad[i];
    float p = param[i];
    if (wd != 0.f) g = g + wd * p;
    if (op == 0) {
      p = p - lr * g;
    } else if (op == 1) {
      const float v = beta1 * s1[i] - lr * g;
      s1[i] = v;
      p = p + v;
    } else {
      const float m = beta1 * s1[i] + (1.f - beta1) * g;
      const float v = beta2 * s2[i] + (1.f - beta2) * g * g;
      s1[i] = m;
      s2[i] = v;
      p = p - lr * (m * mh) / (sqrtf(v * vh) + eps);
    }
    param[i] = p;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void fill_kernel(typename Elem<T>::storage* __restrict__ y, long n, float v,
                                                   int vec) {
  using S = typename Elem<T>::storage;
  constexpr int VE = 16 / sizeof(S);
  const S e = Elem<T>::from_f32(v);
  const long nv = vec ? n / VE : 0;
  if (nv) {
    S chunk[VE];
#pragma unroll
    for (int j = 0; j < VE; ++j) chunk[j] = e;
    const uint4 c = *reinterpret_cast<const uint4*>(chunk);
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < nv; i += (long)gridDim.x * 256)
      reinterpret_cast<uint4*>(y)[i] = c;
  }
  for (long i = nv * VE + (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) y[i] = e;
}

// ============================================================== typed launchers
template <typename T>
int run_direct_fwd(const void* x, const void* w, const void* bias, void* y, const ConvGeom& g, hipStream_t st,
                   int act) {
  long total = (long)g.N * g.O * g.P * g.Q;
  using S = typename Elem<T>::storage;
  // few products per output: the block-per-(image, 8 channels) kernel (same sums, same bits)
  const bool rs_ok = g.R == g.S && (g.R == 1 || g.R == 3 || g.R == 5);
  if (rs_ok && (long)g.C * g.R * g.S <= 128 && g.N <= 65535 && (long)g.P * g.Q < (1L << 31) &&
      (long)g.C * g.H * g.W < (1L << 31)) {
    dim3 grid((unsigned)g.N, (unsigned)((g.O + 7) / 8), (unsigned)std::min<long>(((long)g.P * g.Q + 255) / 256, 64));
    if (g.R == 3)
      direct_fwd_small_kernel<T, 3, 3, 8><<<grid, 256, 0, st>>>((const S*)x, (const S*)w, (const S*)bias, (S*)y, g, act);
    else if (g.R == 5)
      direct_fwd_small_kernel<T, 5, 5, 8><<<grid, 256, 0, st>>>((const S*)x, (const S*)w, (const S*)bias, (S*)y, g, act);
    else
      direct_fwd_small_kernel<T, 1, 1, 8><<<grid, 256, 0, st>>>((const S*)x, (const S*)w, (const S*)bias, (S*)y, g, act);
    VH_LAUNCH_CHECK();
    return VH_OK;
  }
  direct_fwd_kernel<T><<<grid_for(total), 256, 0, st>>>((const S*)x, (const S*)w, (const S*)bias, (S*)y, g, total,
                                                        act);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <typename T>
int run_direct_dgrad(const void* dy, const void* w, void* dx, const ConvGeom& g, hipStream_t st) {
  long total = (long)g.N * g.C * g.H * g.W;
  using S = typename Elem<T>::storage;
  direct_dgrad_kernel<T><<<grid_for(total), 256, 0, st>>>((const S*)dy, (const S*)w, (S*)dx, g, total);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

// Forward of the same geometry seen from the other side (fp32): y[n][o][p][q] =
// sum over (c, r, s) of x[n][c][2p - 1 + r][2q - 1 + s] w[o][c][r][s] with at
// most 4 input channels and 64 output channels (the input gradient of the
// up-sampling ConvTranspose2d layer), on v_mfma_f32_32x32x2f32: rows o, columns
// the 128 positions of 4 output rows x 32 columns, K = (c, r, s) = 16 C.  A
// block stages the weights [o][k] and the 10 x rows its positions read (zeros
// outside the image) in LDS; wave w takes o 32 (w >> 1) .. + 31 and the 64
// positions of output rows 2 (w & 1), 2 (w & 1) + 1.
constexpr int kCfXP = 76;  // x row pitch (12 * row mod 64 spreads the rows' banks)
constexpr int kCfWP = 66;  // weight row pitch (k and k + 1 on even / odd banks)

__global__ __launch_bounds__(256) void cell_fwd_f32_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           const float* __restrict__ bias, float* __restrict__ y,
                                                           ConvGeom g, int nseg, int tiles, int act) {
  __shared__ __attribute__((aligned(16))) float xs[4 * 10 * kCfXP];
  __shared__ __attribute__((aligned(16))) float wsh[64 * kCfWP];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int C = g.C, O = g.O, K = C * 16;
  const int t = blockIdx.x;
  if (t >= tiles) return;
  const int seg = t % nseg, rest = t / nseg;
  const int prt = g.P / 4 + (g.P % 4 != 0);
  const int p0 = (rest % prt) * 4, img = rest / prt;
  const long HW = (long)g.H * g.W;
  // every load of the prologue is issued before its LDS stores: the weights
  // [o][k] (K % 4 == 0: float4 units, at most 1024 = 4 per thread; rows past O
  // zero) and x rows 2 p0 - 1 .. 2 p0 + 8, columns 64 seg - 4 + 4j (18 float4
  // chunks per row, at most 720 = 3 per thread; zeros outside the image)
  float4 wv[4], xv[3];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = tid + u * 256;
    wv[u] = i < O * K / 4 ? reinterpret_cast<const float4*>(w)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    const int i = tid + u * 256;
    xv[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (i < C * 10 * 18) {
      const int row = i / 18, j = i - row * 18;
      const int c = row / 10, e = row - c * 10;
      const int h = 2 * p0 - 1 + e, col = seg * 64 - 4 + 4 * j;
      if (h >= 0 && h < g.H && col >= 0 && col < g.W)
        xv[u] = *reinterpret_cast<const float4*>(x + ((long)img * C + c) * HW + (long)h * g.W + col);
    }
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = tid + u * 256;
    if (i < 64 * K / 4) {  // rows o >= O get the zeros loaded for them
      const int o = i / (K / 4), k = (i - o * (K / 4)) * 4;
      *reinterpret_cast<float2*>(&wsh[o * kCfWP + k]) = make_float2(wv[u].x, wv[u].y);
      *reinterpret_cast<float2*>(&wsh[o * kCfWP + k + 2]) = make_float2(wv[u].z, wv[u].w);
    }
  }
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    const int i = tid + u * 256;
    if (i < C * 10 * 18) {
      const int row = i / 18, j = i - row * 18;
      *reinterpret_cast<float4*>(&xs[row * kCfXP + 4 * j]) = xv[u];
    }
  }
  __syncthreads();
  const int om = (wave >> 1) * 32, pr0 = (wave & 1) * 2;
  const int fr = lane & 31, fk = lane >> 5;
  f32x16 acc[2] = {f32x16{}, f32x16{}};
  const float* wa = wsh + (om + fr) * kCfWP + fk;
  // column j of the wave: output row pr0 + j, column fr of the segment
  for (int kk = 0; kk < K; kk += 2) {
    const int c = kk >> 4, r = (kk >> 2) & 3, s0 = kk & 3;  // k = kk + fk: s = s0 + fk
    const float a = wa[kk];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float b = xs[(c * 10 + 2 * (pr0 + j) + r) * kCfXP + 2 * fr + 3 + s0 + fk];
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[j], 0, 0, 0);
    }
  }
  const long PQ = (long)g.P * g.Q;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int p = p0 + pr0 + j;
    if (p >= g.P) continue;
    const long base = (long)img * O * PQ + (long)p * g.Q + seg * 32 + fr;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int o = om + (v >> 2) * 8 + fk * 4 + (v & 3);
      if (o < O) {
        float val = acc[j][v] + (bias ? bias[o] : 0.f);
        if (act == 1) val = fmaxf(val, 0.f);
        y[base + (long)o * PQ] = val;
      }
    }
  }
}

// Envelope of cell_fwd_f32: 4x4 taps, stride 2, padding 1, H = 2P, W = 2Q,
// Q % 32 == 0, C <= 4, O <= 64, 16-byte aligned x.
int cell_fwd_f32(const void* x, const void* w, const void* bias, void* y, const ConvGeom& g, int act,
                 hipStream_t st) {
  if (!(g.R == 4 && g.S == 4 && g.sh == 2 && g.sw == 2 && g.ph == 1 && g.pw == 1 && g.C >= 1 && g.C <= 4 &&
        g.O >= 1 && g.O <= 64 && g.Q % 32 == 0 && g.H == 2 * g.P && g.W == 2 * g.Q && act >= 0 && act <= 1 &&
        ((((uintptr_t)x) | ((uintptr_t)w)) & 15) == 0))
    return VH_ERR_UNSUPPORTED;
  const int nseg = g.Q / 32, prt = (g.P + 3) / 4;
  const long tiles = (long)g.N * prt * nseg;
  if (tiles >= (1L << 31)) return VH_ERR_UNSUPPORTED;
  cell_fwd_f32_kernel<<<(unsigned)tiles, 256, 0, st>>>((const float*)x, (const float*)w, (const float*)bias,
                                                      (float*)y, g, nseg, (int)tiles, act);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

// Few-channel ConvTranspose-shaped weight gradient (fp32): the geometry the
// cell kernels take (4x4 taps, stride 2, padding 1, H = 2P, W = 2Q) with C <= 4,
// O <= 64, Q a multiple of 32 and W of 4, 16-byte aligned operands.
static bool convt_cell_wgrad_ok(const ConvGeom& g, const void* dy, const void* x) {
  return g.R == 4 && g.S == 4 && g.sh == 2 && g.sw == 2 && g.ph == 1 && g.pw == 1 && g.C >= 1 && g.C <= 4 &&
         g.O >= 1 && g.O <= 64 && g.Q % kCwQ == 0 && g.H == 2 * g.P && g.W == 2 * g.Q &&
         ((((uintptr_t)dy) | ((uintptr_t)x)) & 15) == 0 && (long)g.N * g.P * (g.Q / kCwQ) < (1L << 30);
}
static int convt_cell_wgrad_blocks(const ConvGeom& g) {
  const int stages = g.N * g.P * (g.Q / kCwQ);
  const int per = std::max(1, (stages + 511) / 512);
  return (stages + per - 1) / per;
}
size_t convt_cell_wgrad_ws(const ConvGeom& g) {
  if (!(g.R == 4 && g.S == 4 && g.sh == 2 && g.sw == 2 && g.C >= 1 && g.C <= 4 && g.O <= 64 && g.Q % kCwQ == 0))
    return 0;
  return (size_t)convt_cell_wgrad_blocks(g) * (((size_t)g.O * g.C * 16 + g.C + 3) & ~(size_t)3) * sizeof(float);
}
int convt_cell_wgrad_f32(const void* dy, const void* x, void* dw, void* db, const ConvGeom& g, float* ws,
                         size_t ws_bytes, hipStream_t st) {
  if (!convt_cell_wgrad_ok(g, dy, x)) return VH_ERR_UNSUPPORTED;
  const int nseg = g.Q / kCwQ, stages = g.N * g.P * nseg;
  const int per = std::max(1, (stages + 511) / 512), blocks = (stages + per - 1) / per;
  const long nw = (long)g.O * g.C * 16, np = (nw + g.C + 3) & ~3L;
  if ((size_t)blocks * np * sizeof(float) > ws_bytes || ((uintptr_t)ws & 15)) return VH_ERR_UNSUPPORTED;
  convt_cell_wgrad_kernel<<<blocks, 256, 0, st>>>((const float*)dy, (const float*)x, ws, g, nseg, stages, per);
  VH_LAUNCH_CHECK();
  const int lg_g = reduce_vec4_lg_groups(blocks);
  convt_cell_wgrad_reduce_kernel<float><<<reduce_vec4_grid(np, lg_g), 256, 0, st>>>(ws, blocks, np, nw, g.C, lg_g,
                                                                                   (float*)dw, (float*)db);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

bool dgrad_smallc_ok(const ConvGeom& g) { return g.C >= 1 && g.C <= 4 && (long)g.O * g.R * g.S * 4 <= 16384; }

template <typename T>
int run_dgrad_smallc(const void* dy, const void* w, const void* bias, const void* mask, void* dx, const ConvGeom& g,
                     hipStream_t st) {
  if (!dgrad_smallc_ok(g)) return VH_ERR_UNSUPPORTED;
  using S = typename Elem<T>::storage;
  const long total = (long)g.N * g.H * g.W;
  const int cc = g.C <= 1 ? 1 : g.C <= 2 ? 2 : 4;
  const size_t lds = (size_t)g.O * g.R * g.S * cc * sizeof(float);
  // 4x4 taps at stride 2, padding 1 (the up-sampling ConvTranspose2d layer):
  // the cell kernel, when a dY row splits into aligned 4-wide loads
  if (g.R == 4 && g.S == 4 && g.sh == 2 && g.sw == 2 && g.ph == 1 && g.pw == 1 && g.Q % 4 == 0 &&
      (reinterpret_cast<uintptr_t>(dy) % (4 * sizeof(S))) == 0 && (reinterpret_cast<uintptr_t>(w) % 4) == 0) {
    const int nct = (g.H + 1) / 2, ncq = ((g.W + 1) / 2 + 3) / 4;
    const long nlanes = (long)g.N * nct * ncq, nblk = (nlanes + 63) / 64;
    // dY addressed by 32-bit buffer offsets, below the out-of-range marker
    if (nblk < (1L << 31) && (long)g.N * g.O * g.P * g.Q * (long)sizeof(S) < (1L << 31) - 16) {
#define VH_CELL(CV)                                                                                           \
  dgrad_cell_kernel<T, CV, 4, 4, 2, 2, 1, 1><<<(unsigned)nblk, 256, 0, st>>>(                                  \
      (const S*)dy, (const S*)w, (const S*)bias, (const S*)mask, (S*)dx, g, ncq, nct, nlanes)
      switch (g.C) {
        case 1: VH_CELL(1); break;
        case 2: VH_CELL(2); break;
        case 3: VH_CELL(3); break;
        default: VH_CELL(4); break;
      }
#undef VH_CELL
      VH_LAUNCH_CHECK();
      return VH_OK;
    }
  }
  const int grid = grid_for(total);
#define VH_SMALLC(CCV)                                                                                        \
  dgrad_smallc_kernel<T, CCV><<<grid, 256, lds, st>>>((const S*)dy, (const S*)w, (const S*)bias, (const S*)mask, \
                                                      (S*)dx, g, total)
  if (cc == 1) VH_SMALLC(1);
  else if (cc == 2) VH_SMALLC(2);
  else VH_SMALLC(4);
#undef VH_SMALLC
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <typename T>
int run_channel_bias_add(void* y, const void* bias, long N, int C, long HW, hipStream_t st) {
  using S = typename Elem<T>::storage;
  const long total = N * C * HW;
  if (total == 0) return VH_OK;
  channel_bias_add_kernel<T><<<grid_for(total), 256, 0, st>>>((S*)y, (const S*)bias, C, HW, total);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

// direct_wgrad_ob_kernel: positions per lane and slices
constexpr int kWgradObIt = 4;
static bool direct_wgrad_ob_ok(const ConvGeom& g) {
  return direct_wgrad_taps_ok(g) && g.R <= 3 && g.O >= 8 && g.C <= 65535 &&
         ((long)g.N * g.P * g.Q + 256 * kWgradObIt - 1) / (256 * kWgradObIt) <= 65535;
}

template <typename T>
size_t direct_wgrad_ws(const ConvGeom& g, int* slices, int* slice_len) {
  long npos = (long)g.N * g.P * g.Q;
  long nw = (long)g.O * g.C * g.R * g.S;
  if (direct_wgrad_ob_ok(g)) {
    *slice_len = 256 * kWgradObIt;
    *slices = (int)((npos + *slice_len - 1) / *slice_len);
    return (size_t)(*slices) * (nw + g.O) * sizeof(float);
  }
  if (direct_wgrad_taps_ok(g)) {
    const int sl = direct_wgrad_taps_slices(g);
    *slice_len = (int)((npos + sl - 1) / sl);
    *slices = (int)((npos + *slice_len - 1) / *slice_len);
    return (size_t)(*slices) * (nw + g.O) * sizeof(float);  // + the bias partials
  }
  int sl = (int)std::min<long>(std::max<long>(1, (2048 + nw - 1) / nw), std::max<long>(1, npos / 1024));
  sl = std::min(sl, 1024);
  int len = (int)((npos + sl - 1) / sl);
  *slices = (int)((npos + len - 1) / len);
  *slice_len = len;
  return (size_t)(*slices) * nw * sizeof(float);
}

template <typename T>
int run_direct_wgrad(const void* dy, const void* x, void* dw, const ConvGeom& g, float* ws, int slices,
                     int slice_len, hipStream_t st, void* db, bool* db_done) {
  using S = typename Elem<T>::storage;
  long nw = (long)g.O * g.C * g.R * g.S;
  if (db_done) *db_done = false;
  if (direct_wgrad_ob_ok(g)) {
    if (db_done) *db_done = db != nullptr;
    float* bp = db ? ws + (long)slices * nw : nullptr;
    dim3 grid((unsigned)((g.O + 7) / 8), (unsigned)g.C, (unsigned)slices);
    if (g.R == 3)
      direct_wgrad_ob_kernel<T, 3, 3, 8, kWgradObIt><<<grid, 256, 0, st>>>((const S*)dy, (const S*)x, ws, g, bp);
    else
      direct_wgrad_ob_kernel<T, 1, 1, 8, kWgradObIt><<<grid, 256, 0, st>>>((const S*)dy, (const S*)x, ws, g, bp);
    VH_LAUNCH_CHECK();
    const int nbw = reduce_splits_grid(nw), nbb = db ? reduce_splits_grid(g.O) : 0;
    direct_wgrad_reduce_kernel<T><<<nbw + nbb, 256, 0, st>>>(ws, slices, nw, g.O, (S*)dw, (S*)db, nbw);
    VH_LAUNCH_CHECK();
    return VH_OK;
  }
  if (direct_wgrad_taps_ok(g)) {
    if (db_done) *db_done = db != nullptr;
    // the bias partials ride along (dB of the same pass, one reduction launch)
    float* bp = db ? ws + (long)slices * nw : nullptr;
    dim3 grid((unsigned)(g.O * g.C), (unsigned)slices);
    if (g.R == 3)
      direct_wgrad_taps_kernel<T, 3, 3><<<grid, 256, 0, st>>>((const S*)dy, (const S*)x, ws, g, slice_len, bp);
    else if (g.R == 5)
      direct_wgrad_taps_kernel<T, 5, 5><<<grid, 256, 0, st>>>((const S*)dy, (const S*)x, ws, g, slice_len, bp);
    else
      direct_wgrad_taps_kernel<T, 1, 1><<<grid, 256, 0, st>>>((const S*)dy, (const S*)x, ws, g, slice_len, bp);
    VH_LAUNCH_CHECK();
    const int nbw = reduce_splits_grid(nw), nbb = db ? reduce_splits_grid(g.O) : 0;
    direct_wgrad_reduce_kernel<T><<<nbw + nbb, 256, 0, st>>>(ws, slices, nw, g.O, (S*)dw, (S*)db, nbw);
    VH_LAUNCH_CHECK();
    return VH_OK;
  } else {
    dim3 grid((unsigned)nw, (unsigned)slices);
    direct_wgrad_kernel<T><<<grid, 256, 0, st>>>((const S*)dy, (const S*)x, ws, g, slice_len);
  }
  VH_LAUNCH_CHECK();
  sum_partials_kernel<T><<<reduce_splits_grid(nw), 256, 0, st>>>(ws, slices, nw, (S*)dw);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <typename T>
int run_pad(const void* x, void* xp, int B, int C, int H, int W, int ph, int pw, hipStream_t st) {
  using S = typename Elem<T>::storage;
  long total = (long)B * C * (H + 2 * ph) * (W + 2 * pw);
  pad_kernel<T><<<grid_for(total), 256, 0, st>>>((const S*)x, (S*)xp, B * C, H, W, ph, pw, total);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <typename T>
int run_crop(const void* xp, void* x, int B, int C, int H, int W, int ph, int pw, hipStream_t st) {
  using S = typename Elem<T>::storage;
  long total = (long)B * C * H * W;
  crop_kernel<T><<<grid_for(total), 256, 0, st>>>((const S*)xp, (S*)x, H, W, ph, pw, total);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <typename T>
int run_im2col(const void* x, void* col, int B, int C, int H, int W, int KH, int KW, int SH, int SW, int HO,
               int WO, hipStream_t st) {
  using S = typename Elem<T>::storage;
  long total = (long)B * HO * WO * C * KH * KW;
  im2col_kernel<T><<<grid_for(total), 256, 0, st>>>((const S*)x, (S*)col, C, H, W, KH, KW, SH, SW, HO, WO, total);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <typename T>
int run_col2im(const void* col, void* x, int B, int C, int H, int W, int KH, int KW, int SH, int SW, int HO,
               int WO, hipStream_t st) {
  using S = typename Elem<T>::storage;
  long total = (long)B * C * H * W;
  col2im_kernel<T><<<grid_for(total), 256, 0, st>>>((const S*)col, (S*)x, C, H, W, KH, KW, SH, SW, HO, WO, total);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <typename T>
int run_col2im_t(const float* dcolT, void* x, int B, int C, int H, int W, int KH, int KW, int SH, int SW, int PH,
                 int PW, int HO, int WO, hipStream_t st) {
  using S = typename Elem<T>::storage;
  long total = (long)B * C * H * W;
  col2im_t_kernel<T><<<grid_for(total), 256, 0, st>>>(dcolT, (S*)x, C, H, W, KH, KW, SH, SW, PH, PW, HO, WO,
                                                      (long)B * HO * WO, total);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <typename T>
int run_relayout_phase(const void* w, void* dst, int O, int C, int R, int S, int sh, int sw, const PhaseTable& tab,
                       hipStream_t st) {
  using E = typename Elem<T>::storage;
  const long total = (long)O * C * R * S;
  if (total <= 0) return VH_OK;
  // rows kernel: enough rows to fill the chip (measured: 512 x 256 rows 18.3 ->
  // 10.2 us; 128 x 64 rows are too few threads, 4.9 -> 5.8 us)
  if (R * S <= 64 && (long)O * C >= 65536 && (R * S % 4 || ((uintptr_t)w & 15) == 0)) {
    PhaseTaps taps{};
    for (int kh = 0; kh < R; ++kh)
      for (int kw = 0; kw < S; ++kw) {
        int pi = 0;
        while (pi < tab.n && (tab.kh0[pi] != kh % sh || tab.kw0[pi] != kw % sw)) ++pi;
        // a tap in no listed phase is not copied (as in the element-wise map)
        taps.tap[kh * S + kw] = pi == tab.n ? -1 : pi | (kh / sh) << 8 | (kw / sw) << 16;
      }
    relayout_phase_rows_kernel<T><<<grid_for((long)O * C), 256, 0, st>>>((const E*)w, (E*)dst, O, C, R * S, tab,
                                                                         taps);
  } else {
    relayout_phase_kernel<T><<<grid_for(total), 256, 0, st>>>((const E*)w, (E*)dst, O, C, R, S, sh, sw, tab);
  }
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <typename T>
int run_relayout(const void* src, void* dst, int A, int B, int RS, int swap, hipStream_t st, int flip) {
  using S = typename Elem<T>::storage;
  if (RS > 64) {
    relayout_simple_kernel<T><<<grid_for((long)A * B * RS), 256, 0, st>>>(
        (const S*)src, (S*)dst, A, B, RS, swap, flip, FastDiv((uint32_t)RS), FastDiv((uint32_t)(swap ? A : B)));
    VH_LAUNCH_CHECK();
    return VH_OK;
  }
  const int R1 = swap ? A : B, R2 = swap ? B * RS : RS, batch = swap ? 1 : A;
  const int TJ = std::min(R2, (64 / RS) * RS);
  dim3 grid((unsigned)((R2 + TJ - 1) / TJ), (unsigned)((R1 + 15) / 16), (unsigned)batch);
  if (grid.z > 65535u) return set_error(VH_ERR_UNSUPPORTED, "too many weight rows for the relayout");
  if (R1 <= 16) {
    relayout_kernel<16, T><<<grid, 256, 0, st>>>((const S*)src, (S*)dst, R1, R2, RS, flip, TJ);
  } else {
    // 32-row tiles: enough blocks for the single-batch (swap) form
    grid.y = (unsigned)((R1 + 31) / 32);
    relayout_kernel<32, T><<<grid, 256, 0, st>>>((const S*)src, (S*)dst, R1, R2, RS, flip, TJ);
  }
  VH_LAUNCH_CHECK();
  return VH_OK;
}

// Slices per plane for the plane-vectorised channel sum (0: not applicable):
// about 4096 blocks in all, each slice at least 1024 chunks of 16 bytes.
static int channel_sum_plane_slices(int N, int C, int HW, size_t esize) {
  const int ve = (int)(16 / esize);
  if (HW % ve || N < 1 || N > 65535 || (long)N * C * HW >= (1L << 31)) return 0;
  const int hwv = HW / ve;
  const long blocks = (long)N * C;
  int hsl = (int)std::max<long>(1, std::min<long>(4096 / std::max<long>(blocks, 1), hwv / 1024));
  return std::min(hsl, 65535);
}

// Short planes (under 128 16-byte chunks, where a block per plane leaves most
// lanes idle): column sums of the [N][C * HW] matrix over slices of rows_per
// images, 16 bytes per lane, then per-channel segment sums.  Returns the slice
// count, 0 when the shape does not qualify.
static int channel_rows_slices(int N, int C, int HW, size_t esize, int* rows_per) {
  const int ve = (int)(16 / esize);
  const long L = (long)C * HW;
  if (N < 1 || HW % ve || HW / ve >= 128 || L >= (1L << 31) || (long)N * L >= (1L << 40)) return 0;
  const long cb = (L / ve + 255) / 256;  // column blocks per slice
  const int s = (int)std::max<long>(1, std::min<long>(N / 8, std::max<long>(1, 512 / cb)));
  *rows_per = (N + s - 1) / s;
  return (N + *rows_per - 1) / *rows_per;
}

size_t channel_sum_ws(int N, int C, int HW, int* nslice) {
  int rp;
  const size_t rows_ws = (size_t)std::max(channel_rows_slices(N, C, HW, 2, &rp), channel_rows_slices(N, C, HW, 4, &rp)) *
                         C * HW * sizeof(float);
  long len = (long)N * HW;
  int s = (int)std::max<long>(1, std::min<long>(std::max<long>(1, 1024 / std::max(C, 1)), len / 4096));
  // the plane-vectorised form keeps N * slices partials (bounded by the larger of the two)
  const int hsl = std::max(channel_sum_plane_slices(N, C, HW, 2), channel_sum_plane_slices(N, C, HW, 4));
  const int sp = hsl ? N * hsl : 0;
  *nslice = s;
  return std::max((size_t)std::max(s, sp) * C * sizeof(float), rows_ws);
}

template <typename T>
int run_channel_sum(const void* x, int N, int C, int HW, void* out, float* ws, int nslice, hipStream_t st) {
  using S = typename Elem<T>::storage;
  {
    int rp;
    const int rs = channel_rows_slices(N, C, HW, sizeof(S), &rp);
    if (rs && (((uintptr_t)x | (uintptr_t)ws) & 15) == 0) {
      constexpr int VE = 16 / sizeof(S);
      const int L = C * HW;
      column_sum_vec_kernel<T><<<dim3((L / VE + 255) / 256, rs), 256, 0, st>>>((const S*)x, N, L, ws, rp);
      VH_LAUNCH_CHECK();
      channel_segment_sum_kernel<T><<<C, 256, 0, st>>>(ws, rs, C, HW, FastDiv((uint32_t)HW), (S*)out);
      VH_LAUNCH_CHECK();
      return VH_OK;
    }
  }
  const int hsl = ((uintptr_t)x & 15) ? 0 : channel_sum_plane_slices(N, C, HW, sizeof(S));
  if (hsl) {
    channel_sum_planes_kernel<T><<<dim3(C, N, hsl), 256, 0, st>>>((const S*)x, C, HW / (int)(16 / sizeof(S)), hsl,
                                                                   ws);
    VH_LAUNCH_CHECK();
    sum_partials_kernel<T><<<reduce_splits_grid(C), 256, 0, st>>>(ws, N * hsl, C, (S*)out);
    VH_LAUNCH_CHECK();
    return VH_OK;
  }
  channel_sum_kernel<T><<<dim3(C, nslice), 256, 0, st>>>((const S*)x, N, C, HW, ws, nslice);
  VH_LAUNCH_CHECK();
  sum_partials_kernel<T><<<reduce_splits_grid(C), 256, 0, st>>>(ws, nslice, C, (S*)out);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

size_t column_sum_ws(int M, int N, int* nslice, int* rows_per) {
  // slices of at least 8 rows, enough of them for ~512 blocks of the
  // 8-columns-per-lane kernel
  int cb = (N + 2047) / 2048;
  int s = std::max(1, std::min(M / 8, std::max(1, 512 / cb)));
  *rows_per = (M + s - 1) / s;
  *nslice = (M + *rows_per - 1) / *rows_per;
  return (size_t)(*nslice) * N * sizeof(float);
}

// out[i] = sum over z of part[z][i] in split order (i < n): the float4 split-group
// kernel when n % 4 == 0 and the slabs are 16-byte aligned, else one output per lane.
template <typename T>
int run_sum_partials(const float* part, int splits, long n, void* out, hipStream_t st) {
  using S = typename Elem<T>::storage;
  if (n % 4 == 0 && ((uintptr_t)part & 15) == 0) {
    const int lg_g = reduce_vec4_lg_groups(splits);
    sum_partials_vec4_kernel<T><<<reduce_vec4_grid(n, lg_g), 256, 0, st>>>(part, splits, n, (S*)out, lg_g);
  } else {
    sum_partials_kernel<T><<<reduce_splits_grid(n), 256, 0, st>>>(part, splits, n, (S*)out);
  }
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <typename T>
int run_column_sum(const void* x, int M, int N, void* out, float* ws, int nslice, int rows_per, hipStream_t st) {
  using S = typename Elem<T>::storage;
  constexpr int VE = 16 / sizeof(S);
  if (N % VE == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)ws & 15) == 0) {
    column_sum_vec_kernel<T><<<dim3((N / VE + 255) / 256, nslice), 256, 0, st>>>((const S*)x, M, N, ws, rows_per);
    VH_LAUNCH_CHECK();
    return run_sum_partials<T>(ws, nslice, N, out, st);
  }
  column_sum_kernel<T><<<dim3((N + 255) / 256, nslice), 256, 0, st>>>((const S*)x, M, N, ws, rows_per);
  VH_LAUNCH_CHECK();
  sum_partials_kernel<T><<<reduce_splits_grid(N), 256, 0, st>>>(ws, nslice, N, (S*)out);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <typename T>
int run_pixel_shuffle(const void* in, void* out, int B, int C, int H, int W, int r, int backward,
                      hipStream_t st) {
  using S = typename Elem<T>::storage;
  long total = (long)B * C * H * W * r * r;
  constexpr int VE = 16 / sizeof(S);
  const bool aligned = (((uintptr_t)in | (uintptr_t)out) & 15) == 0;
  if (aligned && r >= 2 && r <= 4 && W % VE == 0 && total < (1L << 31) && total > 0) {
    const int items = (int)((long)B * C * H * r * (W / VE));
    const int grid = (items + 255) / 256;
    if (r == 2)
      pixel_shuffle_vec_kernel<T, 2><<<grid, 256, 0, st>>>((const S*)in, (S*)out, H, W, items, backward);
    else if (r == 3)
      pixel_shuffle_vec_kernel<T, 3><<<grid, 256, 0, st>>>((const S*)in, (S*)out, H, W, items, backward);
    else
      pixel_shuffle_vec_kernel<T, 4><<<grid, 256, 0, st>>>((const S*)in, (S*)out, H, W, items, backward);
    VH_LAUNCH_CHECK();
    return VH_OK;
  }
  pixel_shuffle_kernel<T><<<grid_for(total), 256, 0, st>>>((const S*)in, (S*)out, C, H, W, r, total, backward);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <typename T>
int run_relu(const void* x, const void* g, void* y, long n, hipStream_t st) {
  using S = typename Elem<T>::storage;
  if (n <= 0) return VH_OK;
  const bool vec = ((((uintptr_t)x | (uintptr_t)y | (uintptr_t)g) & 15) == 0);
  relu_kernel<T><<<grid_for(vec ? n / (16 / (long)sizeof(S)) + 1 : n), 256, 0, st>>>((const S*)x, (const S*)g, (S*)y,
                                                                                      n, vec ? 1 : 0);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

size_t sum_ws_bytes(long n) { return (size_t)std::max<long>(1, std::min<long>(1024, (n + 4095) / 4096)) * 4; }

template <typename T>
int run_sum(const void* x, long n, float* out, float* ws, hipStream_t st) {
  using S = typename Elem<T>::storage;
  const int nb = (int)std::max<long>(1, std::min<long>(1024, (n + 4095) / 4096));
  constexpr long VE = 16 / sizeof(S);
  const bool vec = ((uintptr_t)x & 15) == 0;
  long per = std::max<long>(1, (n + nb - 1) / nb);
  if (vec) per = (per + VE - 1) / VE * VE;  // slices start on 16-byte boundaries
  const int nb2 = (int)((n + per - 1) / per);
  sum_slices_kernel<T><<<std::max(nb2, 1), 256, 0, st>>>((const S*)x, n, per, ws, vec ? 1 : 0);
  VH_LAUNCH_CHECK();
  sum_partials_scalar_kernel<<<1, 256, 0, st>>>(ws, std::max(nb2, 1), out);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <typename T>
int run_fill(void* y, long n, float v, hipStream_t st) {
  using S = typename Elem<T>::storage;
  if (n <= 0) return VH_OK;
  const bool vec = ((uintptr_t)y & 15) == 0;
  fill_kernel<T><<<grid_for(vec ? n / (long)(16 / sizeof(S)) + 1 : n), 256, 0, st>>>((S*)y, n, v, vec ? 1 : 0);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <typename T>
int run_add_inplace(void* a, const void* b, long n, hipStream_t st) {
  using S = typename Elem<T>::storage;
  if (n <= 0) return VH_OK;
  add_inplace_kernel<T><<<grid_for(n), 256, 0, st>>>((S*)a, (const S*)b, n);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

int run_cast(int from, int to, const void* src, void* dst, long n, hipStream_t st) {
  if (n <= 0) return VH_OK;
  if (from == to) {
    VH_HIP_CHECK(hipMemcpyAsync(dst, src, (size_t)n * (from == VH_BF16 ? 2 : 4), hipMemcpyDeviceToDevice, st));
    return VH_OK;
  }
  if (from == VH_F32)
    cast_kernel<float, bf16><<<grid_for(n), 256, 0, st>>>((const float*)src, (uint16_t*)dst, n);
  else
    cast_kernel<bf16, float><<<grid_for(n), 256, 0, st>>>((const uint16_t*)src, (float*)dst, n);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <typename T>
int run_batched_transpose(const void* in, void* out, int B, int R, int Cc, hipStream_t st) {
  using S = typename Elem<T>::storage;
  if ((long)B * R * Cc <= 0) return VH_OK;
  if ((R + 31) / 32 > 65535 || B > 65535) return set_error(VH_ERR_UNSUPPORTED, "layout transform too large");
  dim3 grid((unsigned)((Cc + 31) / 32), (unsigned)((R + 31) / 32), (unsigned)B);
  batched_transpose_kernel<T><<<grid, 256, 0, st>>>((const S*)in, (S*)out, R, Cc);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

int run_optimizer_step(int op, float lr, float beta1, float beta2, float t, float eps, float wd, float* param,
                       const float* grad, float* s1, float* s2, long n, hipStream_t st) {
  if (n <= 0) return VH_OK;
  // the bias-correction factors are per step, not per element: computed once here
  const float mh = op == 2 ? 1.0f / (1.0f - powf(beta1, t)) : 1.f;
  const float vh = op == 2 ? 1.0f / (1.0f - powf(beta2, t)) : 1.f;
  optimizer_step_kernel<<<grid_for(n), 256, 0, st>>>(param, grad, s1, s2, op, lr, beta1, beta2, mh, vh, eps, wd, n);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

#define VH_INST(T)                                                                                      \
  template int run_direct_fwd<T>(const void*, const void*, const void*, void*, const ConvGeom&, hipStream_t, int); \
  template int run_col2im_t<T>(const float*, void*, int, int, int, int, int, int, int, int, int, int, int, int,  \
                               hipStream_t);                                                            \
  template int run_direct_dgrad<T>(const void*, const void*, void*, const ConvGeom&, hipStream_t);      \
  template int run_dgrad_smallc<T>(const void*, const void*, const void*, const void*, void*,            \
                                   const ConvGeom&, hipStream_t);                                      \
  template int run_channel_bias_add<T>(void*, const void*, long, int, long, hipStream_t);               \
  template size_t direct_wgrad_ws<T>(const ConvGeom&, int*, int*);                                      \
  template int run_direct_wgrad<T>(const void*, const void*, void*, const ConvGeom&, float*, int, int,  \
                                   hipStream_t, void*, bool*);                                          \
  template int run_pad<T>(const void*, void*, int, int, int, int, int, int, hipStream_t);               \
  template int run_crop<T>(const void*, void*, int, int, int, int, int, int, hipStream_t);              \
  template int run_im2col<T>(const void*, void*, int, int, int, int, int, int, int, int, int, int,      \
                             hipStream_t);                                                              \
  template int run_col2im<T>(const void*, void*, int, int, int, int, int, int, int, int, int, int,      \
                             hipStream_t);                                                              \
  template int run_relayout<T>(const void*, void*, int, int, int, int, hipStream_t, int);               \
  template int run_relayout_phase<T>(const void*, void*, int, int, int, int, int, int, const PhaseTable&, \
                                     hipStream_t);                                                      \
  template int run_channel_sum<T>(const void*, int, int, int, void*, float*, int, hipStream_t);         \
  template int run_column_sum<T>(const void*, int, int, void*, float*, int, int, hipStream_t);          \
  template int run_sum_partials<T>(const float*, int, long, void*, hipStream_t);                        \
  template int run_pixel_shuffle<T>(const void*, void*, int, int, int, int, int, int, hipStream_t);     \
  template int run_relu<T>(const void*, const void*, void*, long, hipStream_t);                         \
  template int run_sum<T>(const void*, long, float*, float*, hipStream_t);                              \
  template int run_fill<T>(void*, long, float, hipStream_t);                                            \
  template int run_add_inplace<T>(void*, const void*, long, hipStream_t);                              \
  template int run_batched_transpose<T>(const void*, void*, int, int, int, hipStream_t);
VH_INST(float)
VH_INST(bf16)
#undef VH_INST

}  // namespace vh
