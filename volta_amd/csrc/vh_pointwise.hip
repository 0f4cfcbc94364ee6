// vh_pointwise.hip -- strided 1x1 convolutions (pad 0), bf16 storage, fp32
// accumulation: the ResNet projection shortcut (1x1, stride 2).
//
// All three passes are GEMMs over output positions with a short contraction
// (C or O channels, or the positions themselves for the weight gradient).
// They are HBM-bound (about 21 FLOP per byte at the config-3 shape), so the
// kernels read each operand once, straight from NCHW into MFMA fragments
// (v_mfma_f32_32x32x16_bf16), with no LDS staging and no workspace besides
// the weight-gradient partial sums:
//
//  forward   y[n,o,p,q]   = sum_c W[o,c] x[n,c,p*s,q*s]          (+ bias[o])
//  dgrad     dx[n,c,h,w]  = sum_o W[o,c] dy[n,o,h/s,w/s]  if s | h and s | w, else 0
//  wgrad     dW[o,c]      = sum_{n,p,q} dy[n,o,p,q] x[n,c,p*s,q*s]
//
// Fragment layout of the 32x32x16 MFMA: lane l supplies row / column (l & 31)
// and contraction indices 8*(l >> 5) .. +7; the result element v of lane l is
// row (v >> 2) * 8 + (l >> 5) * 4 + (v & 3), column (l & 31).
#include <algorithm>

#include "vh_common.hpp"
#include "vh_kernels.hpp"

namespace vh {

typedef unsigned int u32x4p __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2p __attribute__((ext_vector_type(2)));

namespace {

constexpr int kOutOfRange = (int)0x80000000u;  // buffer offset past every range: loads 0, stores dropped

struct PwArgs {
  const void* x;      // [B][C][H][W]
  const void* w;      // [O][C] (the dgrad kernel transposes it into LDS)
  const void* dy;     // [B][O][P][Q]
  const uint16_t* bias;
  void* out;          // forward y; dgrad dx
  float* part;        // wgrad partial sums [blocks][O][C]
  int B, C, H, W, O, P, Q, S;
  int npos;           // B*P*Q
  FastDiv fPQ, fQ;
  int x_bytes, w_bytes, dy_bytes, out_bytes;
  int quads_per_block;  // wgrad: stages (4 output rows) per block
  FastDiv fPQ4;         // wgrad: P/4
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, bytes, 0x00020000);
}

__device__ __forceinline__ bf16x8 pack8(const uint16_t (&v)[8]) {
  u32x4p u;
  u[0] = v[0] | ((uint32_t)v[1] << 16);
  u[1] = v[2] | ((uint32_t)v[3] << 16);
  u[2] = v[4] | ((uint32_t)v[5] << 16);
  u[3] = v[6] | ((uint32_t)v[7] << 16);
  return __builtin_bit_cast(bf16x8, u);
}

// even bf16 elements of 8 consecutive ones (x at stride 2 along a row)
__device__ __forceinline__ u32x2p evens(u32x4p v) {
  u32x2p r;
  r[0] = __builtin_amdgcn_perm(v[1], v[0], 0x05040100u);
  r[1] = __builtin_amdgcn_perm(v[3], v[2], 0x05040100u);
  return r;
}

// ------------------------------------------------------------------ forward
// Block: the weight tile W[o0 .. o0+MT*32)[0 .. C) is copied to LDS once (odd
// 16-byte pitch), then each of the 4 waves computes MT*32 output channels for
// PT_FWD tiles of 32 output positions.  B fragment: 8 channels of one position (8
// two-byte loads, channel planes apart); A fragment: one ds_read_b128.
constexpr int PT_FWD = 1;  // position tiles per wave (one: twice the blocks in flight, measured faster)
constexpr int PT_DG = 2;   // position tiles per wave of the input gradient

template <int MT>
__global__ __launch_bounds__(256) void pw_fwd_bf16_kernel(PwArgs a) {
  extern __shared__ __attribute__((aligned(16))) u32x4p wlds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int o0 = blockIdx.y * MT * 32;
  const int CU = a.C / 8, WPU = CU | 1;  // 16-byte units per weight row, LDS pitch
  {
    const __amdgpu_buffer_rsrc_t wr = rsrc(a.w, a.w_bytes);
    for (int u = tid; u < MT * 32 * CU; u += 256) {
      const int r = u / CU, cu = u - r * CU;
      const int o = o0 + r;
      wlds[r * WPU + cu] = __builtin_bit_cast(
          u32x4p, __builtin_amdgcn_raw_buffer_load_b128(wr, o < a.O ? (o * a.C + cu * 8) * 2 : kOutOfRange, 0, 0));
    }
  }
  __syncthreads();
  const int HW2 = a.H * a.W * 2;
  const int PQ = a.P * a.Q;
  const int PQ2 = PQ * 2;
  const __amdgpu_buffer_rsrc_t xr = rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t yr = rsrc(a.out, a.out_bytes);
  for (int t = 0; t < PT_FWD; ++t) {
    const uint32_t pos = (((uint32_t)blockIdx.x * PT_FWD + t) * 4u + (uint32_t)wave) * 32u + (uint32_t)col;
    const bool valid = pos < (uint32_t)a.npos;
    uint32_t n, pq, p, q;
    a.fPQ.divmod(valid ? pos : 0u, n, pq);
    a.fQ.divmod(pq, p, q);
    const int xbase = (int)((n * (uint32_t)a.C * (uint32_t)(a.H * a.W) + p * (uint32_t)(a.S * a.W) +
                             q * (uint32_t)a.S) * 2u) + half * 8 * HW2;
    int xo[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) xo[j] = valid ? xbase + j * HW2 : kOutOfRange;

    f32x16 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x16{};
    for (int c0 = 0; c0 < a.C; c0 += 16) {
      const int so = c0 * HW2;
      uint16_t xv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) xv[j] = __builtin_amdgcn_raw_buffer_load_b16(xr, xo[j], so, 0);
      bf16x8 af[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        af[mt] = __builtin_bit_cast(bf16x8, wlds[(mt * 32 + col) * WPU + (c0 >> 3) + half]);
      const bf16x8 bf = pack8(xv);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mt], bf, acc[mt], 0, 0, 0);
    }

    // epilogue: fp32 bias add, one rounding, NCHW store (lanes walk consecutive positions)
    const int yo = valid ? (int)((n * (uint32_t)a.O * (uint32_t)PQ + pq) * 2u) + half * 4 * PQ2 : kOutOfRange;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int orow = o0 + mt * 32 + (v >> 2) * 8 + (v & 3);
        const int o = orow + half * 4;
        if (o < a.O) {
          const float b = a.bias ? bf16_to_f32(a.bias[o]) : 0.f;
          __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (__bf16)(acc[mt][v] + b)), yr, yo,
                                                orow * PQ2, 0);
        }
      }
  }
}

// Stride 2 with J consecutive output positions per lane (Q % J == 0, W % (2J)
// == 0): one 4J-byte load of 2J input elements gives channel c at J positions,
// so the block's x is read with J times fewer, J times wider loads.  B
// fragment j (j < J) holds position J * (lane & 31) + j of the wave's 32 J
// positions; the J results of an output channel are one 2J-byte store.
template <int MT, int J>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void pw_fwd_vec_bf16_kernel(PwArgs a) {
  static_assert(J == 2 || J == 4, "two or four positions per lane");
  extern __shared__ __attribute__((aligned(16))) u32x4p wlds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int o0 = blockIdx.y * MT * 32;
  const int CU = a.C / 8, WPU = CU | 1;
  {
    const __amdgpu_buffer_rsrc_t wr = rsrc(a.w, a.w_bytes);
    for (int u = tid; u < MT * 32 * CU; u += 256) {
      const int r = u / CU, cu = u - r * CU;
      const int o = o0 + r;
      wlds[r * WPU + cu] = __builtin_bit_cast(
          u32x4p, __builtin_amdgcn_raw_buffer_load_b128(wr, o < a.O ? (o * a.C + cu * 8) * 2 : kOutOfRange, 0, 0));
    }
  }
  __syncthreads();
  const int HW2 = a.H * a.W * 2;
  const int PQ = a.P * a.Q;
  const int PQ2 = PQ * 2;
  const __amdgpu_buffer_rsrc_t xr = rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t yr = rsrc(a.out, a.out_bytes);
  // first of the lane's J positions (all in one output row)
  const uint32_t pos = ((uint32_t)blockIdx.x * 4u + (uint32_t)wave) * (32u * J) + (uint32_t)col * J;
  const bool valid = pos < (uint32_t)a.npos;
  uint32_t n, pq, p, q;
  a.fPQ.divmod(valid ? pos : 0u, n, pq);
  a.fQ.divmod(pq, p, q);
  const int xbase = (int)((n * (uint32_t)a.C * (uint32_t)(a.H * a.W) + p * (uint32_t)(2 * a.W) + q * 2u) * 2u) +
                    half * 8 * HW2;
  int xo[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) xo[e] = valid ? xbase + e * HW2 : kOutOfRange;

  f32x16 acc[MT][J];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < J; ++j) acc[mt][j] = f32x16{};
  for (int c0 = 0; c0 < a.C; c0 += 16) {
    const int so = c0 * HW2;
    // E[e][h]: channel e, positions 2h and 2h + 1 (low, high half)
    uint32_t E[8][J / 2];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if constexpr (J == 2) {
        const u32x2p v = __builtin_bit_cast(u32x2p, __builtin_amdgcn_raw_buffer_load_b64(xr, xo[e], so, 0));
        E[e][0] = __builtin_amdgcn_perm(v[1], v[0], 0x05040100u);
      } else {
        const u32x2p v = evens(__builtin_bit_cast(u32x4p, __builtin_amdgcn_raw_buffer_load_b128(xr, xo[e], so, 0)));
        E[e][0] = v[0];
        E[e][1] = v[1];
      }
    }
    bf16x8 bf[J];
#pragma unroll
    for (int h = 0; h < J / 2; ++h) {
      u32x4p lo, hi;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lo[i] = __builtin_amdgcn_perm(E[2 * i + 1][h], E[2 * i][h], 0x05040100u);
        hi[i] = __builtin_amdgcn_perm(E[2 * i + 1][h], E[2 * i][h], 0x07060302u);
      }
      bf[2 * h] = __builtin_bit_cast(bf16x8, lo);
      bf[2 * h + 1] = __builtin_bit_cast(bf16x8, hi);
    }
    bf16x8 af[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      af[mt] = __builtin_bit_cast(bf16x8, wlds[(mt * 32 + col) * WPU + (c0 >> 3) + half]);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < J; ++j) acc[mt][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mt], bf[j], acc[mt][j], 0, 0, 0);
  }

  // epilogue: fp32 bias add, one rounding, the J positions of a channel in one store
  const int yo = valid ? (int)((n * (uint32_t)a.O * (uint32_t)PQ + pq) * 2u) + half * 4 * PQ2 : kOutOfRange;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int orow = o0 + mt * 32 + (v >> 2) * 8 + (v & 3);
      const int o = orow + half * 4;
      if (o < a.O) {
        const float b = a.bias ? bf16_to_f32(a.bias[o]) : 0.f;
        uint32_t w[J / 2];
#pragma unroll
        for (int h = 0; h < J / 2; ++h)
          w[h] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(acc[mt][2 * h][v] + b)) |
                 ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(acc[mt][2 * h + 1][v] + b)) << 16);
        if constexpr (J == 2) {
          __builtin_amdgcn_raw_buffer_store_b32(w[0], yr, yo, orow * PQ2, 0);
        } else {
          u32x2p w2;
          w2[0] = w[0];
          w2[1] = w[1];
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2p, w2), yr, yo, orow * PQ2, 0);
        }
      }
    }
}

// ------------------------------------------------------------------ input gradient
// Same GEMM shape with rows = input channels (A = W^T [C][O], staged in LDS
// like the forward weights) and contraction over output channels (B = 8
// channels of dY at one position).  Each result is written with the zeros of
// its s x s cell of dX, so dX is covered exactly once (the cells tile
// [0,H) x [0,W) because (P-1)*s <= H-1 < P*s).
template <int MT, bool S2>
__global__ __launch_bounds__(256) void pw_dgrad_bf16_kernel(PwArgs a) {
  extern __shared__ __attribute__((aligned(16))) u32x4p wlds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int c0 = blockIdx.y * MT * 32;
  const int OU = a.O / 8, WPU = OU | 1;
  {
    // A = W^T: the block's rows c0 .. c0+MT*32 of [C][O], transposed on the way
    // into LDS from the layer's W [O][C] (C % 8 == 0): each 16-byte unit of W
    // (8 consecutive c of one o) is scattered down column o of 8 LDS rows
    const __amdgpu_buffer_rsrc_t wr = rsrc(a.w, a.w_bytes);
    uint16_t* w16 = reinterpret_cast<uint16_t*>(wlds);
    constexpr int NCU = MT * 4;  // 8-channel units per block row range
    for (int u = tid; u < a.O * NCU; u += 256) {
      const int cu = u / a.O, o = u - cu * a.O;  // lanes along o: one LDS row per wave
      const int c = c0 + cu * 8;
      const u32x4p v = __builtin_bit_cast(
          u32x4p, __builtin_amdgcn_raw_buffer_load_b128(wr, c < a.C ? (o * a.C + c) * 2 : kOutOfRange, 0, 0));
#pragma unroll
      for (int e = 0; e < 8; ++e)
        w16[(cu * 8 + e) * (WPU * 8) + o] = (uint16_t)((v[e >> 1] >> (16 * (e & 1))) & 0xffffu);
    }
  }
  __syncthreads();
  const int PQ2 = a.P * a.Q * 2;
  const int HW2 = a.H * a.W * 2;
  const __amdgpu_buffer_rsrc_t dr = rsrc(a.dy, a.dy_bytes);
  const __amdgpu_buffer_rsrc_t xr = rsrc(a.out, a.out_bytes);
  for (int t = 0; t < PT_DG; ++t) {
    const uint32_t pos = (((uint32_t)blockIdx.x * PT_DG + t) * 4u + (uint32_t)wave) * 32u + (uint32_t)col;
    const bool valid = pos < (uint32_t)a.npos;
    uint32_t n, pq, p, q;
    a.fPQ.divmod(valid ? pos : 0u, n, pq);
    a.fQ.divmod(pq, p, q);
    const int dbase = (int)((n * (uint32_t)a.O * (uint32_t)(a.P * a.Q) + pq) * 2u) + half * 8 * PQ2;
    int dyo[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) dyo[j] = valid ? dbase + j * PQ2 : kOutOfRange;

    f32x16 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x16{};
    for (int k0 = 0; k0 < a.O; k0 += 16) {
      const int so = k0 * PQ2;
      uint16_t dv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) dv[j] = __builtin_amdgcn_raw_buffer_load_b16(dr, dyo[j], so, 0);
      bf16x8 af[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        af[mt] = __builtin_bit_cast(bf16x8, wlds[(mt * 32 + col) * WPU + (k0 >> 3) + half]);
      const bf16x8 bf = pack8(dv);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mt], bf, acc[mt], 0, 0, 0);
    }

    const int h0 = (int)p * a.S, w0 = (int)q * a.S;
    const int xo = valid ? (int)((n * (uint32_t)a.C * (uint32_t)(a.H * a.W) + (uint32_t)(h0 * a.W + w0)) * 2u) +
                               half * 4 * HW2
                         : kOutOfRange;
    if (S2) {
      // s = 2, W even: (value, 0) as one 4-byte store on row h0, (0, 0) on row h0 + 1
      const int xo1 = (valid && h0 + 1 < a.H) ? xo + a.W * 2 : kOutOfRange;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int crow = c0 + mt * 32 + (v >> 2) * 8 + (v & 3);
          if (crow + half * 4 < a.C) {
            const uint32_t val = __builtin_bit_cast(uint16_t, (__bf16)acc[mt][v]);
            __builtin_amdgcn_raw_buffer_store_b32(val, xr, xo, crow * HW2, 0);
            __builtin_amdgcn_raw_buffer_store_b32(0u, xr, xo1, crow * HW2, 0);
          }
        }
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int crow = c0 + mt * 32 + (v >> 2) * 8 + (v & 3);
          if (crow + half * 4 < a.C) {
            const uint16_t val = __builtin_bit_cast(uint16_t, (__bf16)acc[mt][v]);
            for (int dh = 0; dh < a.S; ++dh)
              for (int dw = 0; dw < a.S; ++dw) {
                const bool in = valid && h0 + dh < a.H && w0 + dw < a.W;
                __builtin_amdgcn_raw_buffer_store_b16((dh | dw) ? (uint16_t)0 : val, xr,
                                                      in ? xo + (dh * a.W + dw) * 2 : kOutOfRange, crow * HW2, 0);
              }
          }
        }
    }
  }
}

// Stride 2, W % 4 == 0, with two dY positions per lane (one 4-byte load per
// output channel): B fragment j (j < 2) holds position 2 * (lane & 31) + j of
// the wave's 64; the two results of an input channel and their zeros are one
// 8-byte store on row 2p and one on row 2p + 1.
template <int MT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void pw_dgrad_vec_bf16_kernel(PwArgs a) {
  extern __shared__ __attribute__((aligned(16))) u32x4p wlds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int c0 = blockIdx.y * MT * 32;
  const int OU = a.O / 8, WPU = OU | 1;
  {
    // A = W^T, as in the one-position kernel
    const __amdgpu_buffer_rsrc_t wr = rsrc(a.w, a.w_bytes);
    uint16_t* w16 = reinterpret_cast<uint16_t*>(wlds);
    constexpr int NCU = MT * 4;
    for (int u = tid; u < a.O * NCU; u += 256) {
      const int cu = u / a.O, o = u - cu * a.O;
      const int c = c0 + cu * 8;
      const u32x4p v = __builtin_bit_cast(
          u32x4p, __builtin_amdgcn_raw_buffer_load_b128(wr, c < a.C ? (o * a.C + c) * 2 : kOutOfRange, 0, 0));
#pragma unroll
      for (int e = 0; e < 8; ++e)
        w16[(cu * 8 + e) * (WPU * 8) + o] = (uint16_t)((v[e >> 1] >> (16 * (e & 1))) & 0xffffu);
    }
  }
  __syncthreads();
  const int PQ2 = a.P * a.Q * 2;
  const int HW2 = a.H * a.W * 2;
  const __amdgpu_buffer_rsrc_t dr = rsrc(a.dy, a.dy_bytes);
  const __amdgpu_buffer_rsrc_t xr = rsrc(a.out, a.out_bytes);
  const uint32_t pos = ((uint32_t)blockIdx.x * 4u + (uint32_t)wave) * 64u + (uint32_t)col * 2u;
  const bool valid = pos < (uint32_t)a.npos;
  uint32_t n, pq, p, q;
  a.fPQ.divmod(valid ? pos : 0u, n, pq);
  a.fQ.divmod(pq, p, q);
  const int dbase = (int)((n * (uint32_t)a.O * (uint32_t)(a.P * a.Q) + pq) * 2u) + half * 8 * PQ2;
  int dyo[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) dyo[e] = valid ? dbase + e * PQ2 : kOutOfRange;

  f32x16 acc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt][0] = acc[mt][1] = f32x16{};
  for (int k0 = 0; k0 < a.O; k0 += 16) {
    const int so = k0 * PQ2;
    uint32_t E[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) E[e] = __builtin_amdgcn_raw_buffer_load_b32(dr, dyo[e], so, 0);
    u32x4p lo, hi;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo[i] = __builtin_amdgcn_perm(E[2 * i + 1], E[2 * i], 0x05040100u);
      hi[i] = __builtin_amdgcn_perm(E[2 * i + 1], E[2 * i], 0x07060302u);
    }
    const bf16x8 bf0 = __builtin_bit_cast(bf16x8, lo), bf1 = __builtin_bit_cast(bf16x8, hi);
    bf16x8 af[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      af[mt] = __builtin_bit_cast(bf16x8, wlds[(mt * 32 + col) * WPU + (k0 >> 3) + half]);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      acc[mt][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mt], bf0, acc[mt][0], 0, 0, 0);
      acc[mt][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mt], bf1, acc[mt][1], 0, 0, 0);
    }
  }

  const int h0 = (int)p * 2, w0 = (int)q * 2;
  const int xo = valid ? (int)((n * (uint32_t)a.C * (uint32_t)(a.H * a.W) + (uint32_t)(h0 * a.W + w0)) * 2u) +
                             half * 4 * HW2
                       : kOutOfRange;
  const int xo1 = (valid && h0 + 1 < a.H) ? xo + a.W * 2 : kOutOfRange;
  u32x2p zero;
  zero[0] = zero[1] = 0u;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int crow = c0 + mt * 32 + (v >> 2) * 8 + (v & 3);
      if (crow + half * 4 < a.C) {
        u32x2p val;
        val[0] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)acc[mt][0][v]);
        val[1] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)acc[mt][1][v]);
        __builtin_amdgcn_raw_buffer_store_b64(val, xr, xo, crow * HW2, 0);
        __builtin_amdgcn_raw_buffer_store_b64(zero, xr, xo1, crow * HW2, 0);
      }
    }
}

// ------------------------------------------------------------------ weight gradient
// s = 2, W % 8 == 0, P % 4 == 0.  The contraction runs over output positions,
// four output rows (4Q positions, never crossing an image) per stage.  A block
// owns 128 output channels x 64 input channels and a range of stages; per
// stage it copies into LDS
//   dY rows  [o][4Q]   (one contiguous 8Q-byte run per o: 16-byte loads), and
//   x rows   [c][4Q]   (the even elements of input rows 2p, 2p+2, ..: 16-byte
//                       loads, 8 bytes kept),
// both K-contiguous with an odd pitch in 16-byte units, so every MFMA fragment
// is one ds_read_b128.  Wave w computes o0 + 32w .. +31 x the block's 64 c.
// The next stage is loaded into registers while the current one is consumed.
// Each block writes one fp32 partial tile [O][C]; a second kernel adds them.
template <int IT>
__global__ __launch_bounds__(256) void pw_wgrad_s2_bf16_kernel(PwArgs a) {
  extern __shared__ __attribute__((aligned(16))) u32x4p lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int o0 = blockIdx.y * 128, c0 = blockIdx.z * 64;
  const int Q = a.Q, PQ = a.P * a.Q, HW = a.H * a.W;
  const int KU = Q / 2;                 // 16-byte units per LDS row (4Q elements)
  const int PU = KU | 1;                // odd pitch
  u32x4p* dys = lds;                    // [128][PU]
  u32x4p* xs = lds + 128 * PU;          // [64][PU]

  // load items, fixed for the block: dY item i -> (o = i / KU, unit u = i % KU);
  // x item i -> (c = i / Q, row g = (i % Q) / (W/8), unit u), W/8 = Q/4 units per row
  const int WU = Q / 4;
  int dy_g[IT], dy_l[IT], x_g[IT], x_l[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int i = tid + it * 256;
    const int o = i / KU, u = i % KU;
    const bool ok = o < 128 && o0 + o < a.O;
    dy_g[it] = ok ? ((o0 + o) * PQ * 2 + u * 16) : kOutOfRange;
    dy_l[it] = o < 128 ? o * PU + u : -1;
    const int c = i / Q, r = i % Q, g = r / WU, xu = r % WU;
    const bool okx = c < 64 && c0 + c < a.C;
    x_g[it] = okx ? ((c0 + c) * HW * 2 + g * 2 * a.W * 2 + xu * 16) : kOutOfRange;
    x_l[it] = c < 64 ? c * PU * 2 + g * WU + xu : -1;  // in 8-byte units (4 positions each)
  }
  const __amdgpu_buffer_rsrc_t dr = rsrc(a.dy, a.dy_bytes);
  const __amdgpu_buffer_rsrc_t xr = rsrc(a.x, a.x_bytes);

  const int stages = a.B * a.P / 4;
  const int s_begin = blockIdx.x * a.quads_per_block;
  const int s_end = min(s_begin + a.quads_per_block, stages);

  u32x4p rdy[IT], rx[IT];
  auto gload = [&](int sidx) {
    uint32_t n, p4;
    a.fPQ4.divmod((uint32_t)sidx, n, p4);  // fPQ4 holds P/4 here
    const int p0 = (int)p4 * 4;
    const int dso = (int)((n * (uint32_t)a.O * (uint32_t)PQ + (uint32_t)(p0 * Q)) * 2u);
    const int xso = (int)((n * (uint32_t)a.C * (uint32_t)HW + (uint32_t)(2 * p0 * a.W)) * 2u);
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      rdy[it] = __builtin_bit_cast(u32x4p, __builtin_amdgcn_raw_buffer_load_b128(
                                              dr, dy_g[it] == kOutOfRange ? kOutOfRange : dy_g[it] + dso, 0, 0));
      rx[it] = __builtin_bit_cast(u32x4p, __builtin_amdgcn_raw_buffer_load_b128(
                                             xr, x_g[it] == kOutOfRange ? kOutOfRange : x_g[it] + xso, 0, 0));
    }
  };
  auto sstore = [&]() {
    u32x2p* xs8 = reinterpret_cast<u32x2p*>(xs);
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      if (dy_l[it] >= 0) dys[dy_l[it]] = rdy[it];
      if (x_l[it] >= 0) xs8[x_l[it]] = evens(rx[it]);
    }
  };

  const int row = lane & 31, half = lane >> 5;
  f32x16 acc[2] = {f32x16{}, f32x16{}};
  if (s_begin < s_end) gload(s_begin);
  for (int sidx = s_begin; sidx < s_end; ++sidx) {
    sstore();
    __syncthreads();
    if (sidx + 1 < s_end) gload(sidx + 1);
    const u32x4p* ap = dys + (wave * 32 + row) * PU + half;
    const u32x4p* bp = xs + row * PU + half;
    for (int k = 0; k < KU; k += 2) {
      const bf16x8 af = __builtin_bit_cast(bf16x8, ap[k]);
      const bf16x8 b0 = __builtin_bit_cast(bf16x8, bp[k]);
      const bf16x8 b1 = __builtin_bit_cast(bf16x8, bp[32 * PU + k]);
      acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, b0, acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, b1, acc[1], 0, 0, 0);
    }
    __syncthreads();
  }

  // partial tile of this block: part[blockIdx.x][o][c]
  float* part = a.part + (size_t)blockIdx.x * a.O * a.C;
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int c = c0 + nt * 32 + row;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int o = o0 + wave * 32 + (v >> 2) * 8 + half * 4 + (v & 3);
      if (o < a.O && c < a.C) part[(size_t)o * a.C + c] = acc[nt][v];
    }
  }
}

bool fits_i32(long v) { return v > 0 && v < (1L << 31) - 16; }

PwArgs base_args(int B, int C, int H, int W, int O, int S) {
  PwArgs a{};
  a.B = B;
  a.C = C;
  a.H = H;
  a.W = W;
  a.O = O;
  a.S = S;
  a.P = (H - 1) / S + 1;
  a.Q = (W - 1) / S + 1;
  a.npos = B * a.P * a.Q;
  a.fPQ = FastDiv((uint32_t)(a.P * a.Q));
  a.fQ = FastDiv((uint32_t)a.Q);
  a.x_bytes = (int)((long)B * C * H * W * 2);
  a.dy_bytes = (int)((long)B * O * a.P * a.Q * 2);
  a.w_bytes = O * C * 2;
  return a;
}

bool envelope(int B, int C, int H, int W, int O, int S) {
  if (S < 2 || B <= 0 || C <= 0 || O <= 0 || H <= 0 || W <= 0) return false;
  const long P = (H - 1) / S + 1, Q = (W - 1) / S + 1;
  return fits_i32((long)B * C * H * W * 2) && fits_i32((long)B * O * P * Q * 2) && fits_i32((long)O * C * 2);
}

}  // namespace

// ------------------------------------------------------------------ host entry points
int pw_conv_bf16_fwd(const void* x, const void* w, const void* bias, void* y, int B, int C, int H, int W, int O,
                     int S, hipStream_t st) {
  if (!envelope(B, C, H, W, O, S) || C % 16 != 0 || C > 248) return VH_ERR_UNSUPPORTED;  // LDS weight tile
  PwArgs a = base_args(B, C, H, W, O, S);
  a.x = x;
  a.w = w;
  a.bias = (const uint16_t*)bias;
  a.out = y;
  a.out_bytes = a.dy_bytes;
  // stride 2 with pairs of output positions per row: the vector form, 128
  // output channels per block (measured: pairs beat both single positions and
  // runs of four on two 64-channel blocks)
  if (S == 2 && a.Q % 2 == 0 && W % 4 == 0 && ((uintptr_t)x & 7) == 0 && ((uintptr_t)y & 3) == 0) {
    dim3 g((a.npos + 4 * 32 * 2 - 1) / (4 * 32 * 2), (O + 127) / 128);
    pw_fwd_vec_bf16_kernel<4, 2><<<g, 256, (size_t)128 * ((C / 8) | 1) * 16, st>>>(a);
    VH_LAUNCH_CHECK();
    return VH_OK;
  }
  dim3 grid((a.npos + PT_FWD * 128 - 1) / (PT_FWD * 128), (O + 127) / 128);
  const size_t lds = (size_t)(O <= 64 ? 64 : 128) * ((C / 8) | 1) * 16;
  if (O <= 64) {
    grid.y = (O + 63) / 64;
    pw_fwd_bf16_kernel<2><<<grid, 256, lds, st>>>(a);
  } else {
    pw_fwd_bf16_kernel<4><<<grid, 256, lds, st>>>(a);
  }
  VH_LAUNCH_CHECK();
  return VH_OK;
}

int pw_conv_bf16_dgrad(const void* dy, const void* w, void* dx, int B, int C, int H, int W, int O, int S,
                       hipStream_t st) {
  if (!envelope(B, C, H, W, O, S) || O % 16 != 0 || O > 248 || C % 8 != 0)  // LDS weight tile, 16-byte W units
    return VH_ERR_UNSUPPORTED;
  PwArgs a = base_args(B, C, H, W, O, S);
  a.dy = dy;
  a.w = w;
  a.out = dx;
  a.out_bytes = a.x_bytes;
  // stride 2, W % 4 == 0: two positions per lane (8-byte stores of value, 0, value, 0)
  if (S == 2 && W % 4 == 0 && ((uintptr_t)dy & 3) == 0 && ((uintptr_t)dx & 7) == 0) {
    const int MT = C <= 64 ? 2 : 4;
    dim3 g((a.npos + 255) / 256, (C + MT * 32 - 1) / (MT * 32));
    const size_t l = (size_t)MT * 32 * ((O / 8) | 1) * 16;
    if (MT == 2) pw_dgrad_vec_bf16_kernel<2><<<g, 256, l, st>>>(a);
    else pw_dgrad_vec_bf16_kernel<4><<<g, 256, l, st>>>(a);
    VH_LAUNCH_CHECK();
    return VH_OK;
  }
  const bool s2 = S == 2 && W % 2 == 0;
  dim3 grid((a.npos + PT_DG * 128 - 1) / (PT_DG * 128), (C + 127) / 128);
  const size_t lds = (size_t)(C <= 64 ? 64 : 128) * ((O / 8) | 1) * 16;
  if (C <= 64) {
    grid.y = (C + 63) / 64;
    if (s2) pw_dgrad_bf16_kernel<2, true><<<grid, 256, lds, st>>>(a);
    else pw_dgrad_bf16_kernel<2, false><<<grid, 256, lds, st>>>(a);
  } else {
    if (s2) pw_dgrad_bf16_kernel<4, true><<<grid, 256, lds, st>>>(a);
    else pw_dgrad_bf16_kernel<4, false><<<grid, 256, lds, st>>>(a);
  }
  VH_LAUNCH_CHECK();
  return VH_OK;
}

static int pw_wgrad_plan(int B, int C, int H, int W, int O, int S, PwArgs* out) {
  if (!envelope(B, C, H, W, O, S) || S != 2 || W % 8 != 0) return 0;
  PwArgs a = base_args(B, C, H, W, O, S);
  if (a.P % 4 != 0 || a.Q > 64) return 0;  // Q = W/2 is a multiple of 4
  const int stages = B * a.P / 4;
  const int tiles = ((O + 127) / 128) * ((C + 63) / 64);
  // about 256 blocks in all, each walking a range of stages
  const int blocks = std::max(1, 256 / tiles);
  a.quads_per_block = std::max(1, (stages + blocks - 1) / blocks);  // stages per block
  a.fPQ4 = FastDiv((uint32_t)(a.P / 4));
  *out = a;
  return (stages + a.quads_per_block - 1) / a.quads_per_block;
}

static size_t pw_wgrad_lds(int Q) { return (size_t)(128 + 64) * ((Q / 2) | 1) * 16; }

size_t pw_conv_bf16_wgrad_ws(int B, int C, int H, int W, int O, int S) {
  PwArgs a;
  const int splits = pw_wgrad_plan(B, C, H, W, O, S, &a);
  return splits ? (size_t)splits * O * C * sizeof(float) : 0;
}

template <int IT>
static int launch_pw_wgrad(const PwArgs& a, dim3 grid, hipStream_t st) {
  auto kern = pw_wgrad_s2_bf16_kernel<IT>;
  VH_LDS_LIMIT_ONCE(kern);
  kern<<<grid, 256, pw_wgrad_lds(a.Q), st>>>(a);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

int pw_conv_bf16_wgrad(const void* dy, const void* x, void* dw, int B, int C, int H, int W, int O, int S,
                       float* ws, size_t ws_bytes, hipStream_t st) {
  PwArgs a;
  const int splits = pw_wgrad_plan(B, C, H, W, O, S, &a);
  if (!splits) return VH_ERR_UNSUPPORTED;
  if (ws_bytes < (size_t)splits * O * C * sizeof(float))
    return set_error(VH_ERR_BAD_ARG, "pointwise wgrad: workspace too small");
  if (((uintptr_t)x & 15) || ((uintptr_t)dy & 15)) return VH_ERR_UNSUPPORTED;
  a.dy = dy;
  a.x = x;
  a.part = ws;
  dim3 grid(splits, (O + 127) / 128, (C + 63) / 64);
  // load items per thread: 128 * Q/2 dY units and 64 * Q x units over 256 threads
  const int it = (64 * a.Q + 255) / 256;
  int r;
  if (it <= 4) r = launch_pw_wgrad<4>(a, grid, st);
  else if (it <= 8) r = launch_pw_wgrad<8>(a, grid, st);
  else if (it <= 12) r = launch_pw_wgrad<12>(a, grid, st);
  else r = launch_pw_wgrad<16>(a, grid, st);
  if (r != VH_OK) return r;
  return run_sum_partials<bf16>(ws, splits, (long)O * C, dw, st);
}

}  // namespace vh
