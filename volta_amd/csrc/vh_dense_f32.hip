// vh_dense_f32.hip -- dense fp32 matrix products (matmul, its gradients,
// Linear) on gfx950 MFMA (v_mfma_f32_32x32x2_f32), fp32 accumulation.
//
// C[M][N] = A . B with either operand stored either way: "K-major" ([rows][K],
// the contraction index contiguous: A[M][K], B[N][K]) or "MN-major" ([K][rows]:
// A stored [K][M], B stored [K][N]).  Every operand tile is a copy of 16-byte
// units into LDS in its stored order; an MFMA operand (one fp32 per lane: row
// l % 32, k = l / 32 of a 32 x 2 slice) is one ds_read_b32 from either layout:
//  * K-major tile [row][k], pitch BK + 2 floats: 32 rows x 34 floats lands the
//    32 lanes of one k on the 32 even banks, those of k + 1 on the odd ones;
//  * MN-major tile [k][row], pitch BM + 32 floats: one k is 32 consecutive
//    banks, the next k the other 32.
// Block: 256 threads (2 x 2 waves), tile BM x 128 (BM = 128 or 64), K in
// stages of 32; two LDS stages and two register sets, the loads of stage k+2
// issued before the MFMAs of stage k.  XCD-aware block order as in vh_dense.hip.
#include <type_traits>

#include "vh_kernels.hpp"

namespace vh {

namespace {

typedef unsigned int u32x4f __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2f __attribute__((ext_vector_type(2)));

constexpr int kOORf = (int)0x80000000u;  // buffer offset past every range: loads 0, stores dropped
constexpr int kGroupMf = 8;               // m-tiles per group of the block order

struct DenseF32Args {
  const float* a;     // [M][lda] (K-major) or [K][lda] (MN-major)
  const float* b;     // [N][ldb] (K-major) or [K][ldb] (MN-major)
  float* c;           // [M][ldc]
  const float* bias;  // [N] or nullptr (added to every row)
  int M, N, K, lda, ldb, ldc;
  int a_bytes, b_bytes, c_bytes;
  int tiles_m, tiles_n;
};

template <int BM, bool AT, bool BT>
struct DenseF32Cfg {
  static constexpr int BN = 128, BK = 32;
  static constexpr int KP = BK + 2;                    // K-major tile pitch (floats)
  static constexpr int mn_pitch(int R) { return R + 32; }  // MN-major tile pitch (floats)
  static constexpr int A_FLOATS = AT ? BK * mn_pitch(BM) : BM * KP;
  static constexpr int B_FLOATS = BT ? BK * mn_pitch(BN) : BN * KP;
  static constexpr int STAGE = A_FLOATS + B_FLOATS;    // floats per LDS stage
  static constexpr int AIT = BM * BK / 4 / 256, BIT = BN * BK / 4 / 256;  // 16-byte load units per thread
  static constexpr int FM = BM / 64, FN = BN / 64;     // 32x32 tiles per wave (waves 2 x 2)
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_f(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, bytes, 0x00020000);
}

template <int BM, bool BIAS, bool AT, bool BT>
__global__ __launch_bounds__(256) void gemm_f32_kernel(DenseF32Args g) {
  using Cfg = DenseF32Cfg<BM, AT, BT>;
  constexpr int BN = Cfg::BN, BK = Cfg::BK, KP = Cfg::KP, FM = Cfg::FM, FN = Cfg::FN, STAGE = Cfg::STAGE;
  constexpr int APM = Cfg::mn_pitch(BM), BPM = Cfg::mn_pitch(BN);
  extern __shared__ __attribute__((aligned(16))) float ldsf[];
  const int tid = (int)threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);
  // logical block -> tile in groups of up to 8 m-tiles (blocks resident on one
  // XCD share A and B slices in its L2)
  const int lb = xcd_block(g.tiles_m * g.tiles_n);
  const int grp = lb / (kGroupMf * g.tiles_n), first_m = grp * kGroupMf;
  const int gm = min(g.tiles_m - first_m, kGroupMf);
  const int in_grp = lb - grp * kGroupMf * g.tiles_n;
  const int m0 = (first_m + in_grp % gm) * BM, n0 = (in_grp / gm) * BN;

  // Load units (4 floats).  K-major: unit u -> row u / 8, k quad u % 8 (8 lanes
  // per 128-byte row segment).  MN-major: unit u -> k row u / (R/4), row quad u % (R/4).
  // Global offsets at k0 = 0 (k0 moves in the scalar offset); the k bound is
  // checked per unit, rows past M / N carry an out-of-range offset.
  int a_off[Cfg::AIT], b_off[Cfg::BIT], a_k[Cfg::AIT], b_k[Cfg::BIT], a_l[Cfg::AIT], b_l[Cfg::BIT];
#pragma unroll
  for (int it = 0; it < Cfg::AIT; ++it) {
    const int u = tid + it * 256;
    if constexpr (AT) {
      const int kr = u / (BM / 4), rq = u % (BM / 4);
      a_k[it] = kr;
      a_off[it] = m0 + rq * 4 < g.M ? (kr * g.lda + m0 + rq * 4) * 4 : kOORf;
      a_l[it] = kr * APM + rq * 4;
    } else {
      const int r = u / 8, kq = u % 8;
      a_k[it] = kq * 4;
      a_off[it] = m0 + r < g.M ? ((m0 + r) * g.lda + kq * 4) * 4 : kOORf;
      a_l[it] = r * KP + kq * 4;
    }
  }
#pragma unroll
  for (int it = 0; it < Cfg::BIT; ++it) {
    const int u = tid + it * 256;
    if constexpr (BT) {
      const int kr = u / (BN / 4), rq = u % (BN / 4);
      b_k[it] = kr;
      b_off[it] = n0 + rq * 4 < g.N ? (kr * g.ldb + n0 + rq * 4) * 4 : kOORf;
      b_l[it] = Cfg::A_FLOATS + kr * BPM + rq * 4;
    } else {
      const int r = u / 8, kq = u % 8;
      b_k[it] = kq * 4;
      b_off[it] = n0 + r < g.N ? ((n0 + r) * g.ldb + kq * 4) * 4 : kOORf;
      b_l[it] = Cfg::A_FLOATS + r * KP + kq * 4;
    }
  }
  const __amdgpu_buffer_rsrc_t ar = rsrc_f(g.a, g.a_bytes), br = rsrc_f(g.b, g.b_bytes);

  u32x4f areg[2][Cfg::AIT], breg[2][Cfg::BIT];
  auto gload = [&](auto SET, int k0) {
    constexpr int s = decltype(SET)::value;
    // k0 as a scalar offset: k0 floats along a K-major row, k0 rows of an MN-major operand
    const int ask = AT ? k0 * g.lda * 4 : k0 * 4, bsk = BT ? k0 * g.ldb * 4 : k0 * 4;
#pragma unroll
    for (int it = 0; it < Cfg::AIT; ++it)  // K % 4 == 0: a K-major unit is all in or all out
      areg[s][it] = __builtin_bit_cast(
          u32x4f, __builtin_amdgcn_raw_buffer_load_b128(ar, k0 + a_k[it] < g.K ? a_off[it] : kOORf, ask, 0));
#pragma unroll
    for (int it = 0; it < Cfg::BIT; ++it)
      breg[s][it] = __builtin_bit_cast(
          u32x4f, __builtin_amdgcn_raw_buffer_load_b128(br, k0 + b_k[it] < g.K ? b_off[it] : kOORf, bsk, 0));
  };
  auto sstore = [&](auto SET, int st) {
    constexpr int s = decltype(SET)::value;
    float* base = ldsf + st * STAGE;
    // K-major rows are 136 bytes apart: two 8-byte stores per unit; MN-major
    // units are 16-byte aligned
#pragma unroll
    for (int it = 0; it < Cfg::AIT; ++it) {
      const u32x4f v = areg[s][it];
      if constexpr (AT) {
        *reinterpret_cast<u32x4f*>(base + a_l[it]) = v;
      } else {
        reinterpret_cast<u32x2f*>(base + a_l[it])[0] = u32x2f{v.x, v.y};
        reinterpret_cast<u32x2f*>(base + a_l[it])[1] = u32x2f{v.z, v.w};
      }
    }
#pragma unroll
    for (int it = 0; it < Cfg::BIT; ++it) {
      const u32x4f v = breg[s][it];
      if constexpr (BT) {
        *reinterpret_cast<u32x4f*>(base + b_l[it]) = v;
      } else {
        reinterpret_cast<u32x2f*>(base + b_l[it])[0] = u32x2f{v.x, v.y};
        reinterpret_cast<u32x2f*>(base + b_l[it])[1] = u32x2f{v.z, v.w};
      }
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};
  const int row_l = lane & 31, k_l = lane >> 5;
  auto compute = [&](int st) {
    const float* at = ldsf + st * STAGE;
    const float* bt = ldsf + st * STAGE + Cfg::A_FLOATS;
#pragma unroll
    for (int ks = 0; ks < BK; ks += 2) {
      float af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = AT ? at[(ks + k_l) * APM + wm + i * 32 + row_l] : at[(wm + i * 32 + row_l) * KP + ks + k_l];
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[j] = BT ? bt[(ks + k_l) * BPM + wn + j * 32 + row_l] : bt[(wn + j * 32 + row_l) * KP + ks + k_l];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  const int nk = (g.K + BK - 1) / BK;
  // invariant at an even stage k: LDS buffer 0 holds stage k, register set 1
  // holds stage k+1 (in flight), set 0 is free
  gload(I0{}, 0);
  if (nk > 1) gload(I1{}, BK);
  __builtin_amdgcn_sched_barrier(0);
  sstore(I0{}, 0);
  __syncthreads();
  int kt = 0;
  for (; kt + 3 < nk; kt += 2) {
    gload(I0{}, (kt + 2) * BK);
    __builtin_amdgcn_sched_barrier(0);
    compute(0);
    __builtin_amdgcn_sched_barrier(0);
    sstore(I1{}, 1);
    __syncthreads();
    gload(I1{}, (kt + 3) * BK);
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
    __builtin_amdgcn_sched_barrier(0);
    sstore(I0{}, 0);
    __syncthreads();
  }
  const int rem = nk - kt;  // 1, 2 or 3 stages left
  if (rem == 3) gload(I0{}, (kt + 2) * BK);
  __builtin_amdgcn_sched_barrier(0);
  compute(0);
  if (rem >= 2) {
    sstore(I1{}, 1);
    __syncthreads();
    compute(1);
    if (rem == 3) {
      sstore(I0{}, 0);
      __syncthreads();
      compute(0);
    }
  }

  // epilogue: (+ bias) row-major fp32 stores, lanes walk columns
  const __amdgpu_buffer_rsrc_t cr = rsrc_f(g.c, g.c_bytes);
  const int half_l = lane >> 5;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int col = n0 + wn + j * 32 + row_l;
    const bool cok = col < g.N;
    const float bv = (BIAS && cok) ? g.bias[col] : 0.f;
    const int voff = cok ? (col + half_l * 4 * g.ldc) * 4 : kOORf;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm + i * 32 + (v >> 2) * 8 + (v & 3);  // + 4 * half_l
        if (row + half_l * 4 < g.M)
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, acc[i][j][v] + bv), cr, voff,
                                                row * g.ldc * 4, 0);
      }
  }
}

bool fits_f(long bytes) { return bytes >= 0 && bytes < (1L << 31) - 64; }

template <int BM, bool BIAS, bool AT, bool BT>
int launch_gemm_f32(const DenseF32Args& a0, hipStream_t st) {
  using Cfg = DenseF32Cfg<BM, AT, BT>;
  auto kern = gemm_f32_kernel<BM, BIAS, AT, BT>;
  const size_t lds = (size_t)2 * Cfg::STAGE * 4;
  VH_LDS_LIMIT_ONCE(kern);
  DenseF32Args a = a0;
  a.tiles_m = (a.M + BM - 1) / BM;
  a.tiles_n = (a.N + Cfg::BN - 1) / Cfg::BN;
  kern<<<dim3((unsigned)(a.tiles_m * a.tiles_n)), 256, lds, st>>>(a);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

// 128 x 128 tiles while that grid gives two blocks per CU, else 64 x 128
template <bool AT, bool BT>
int launch_layout_f32(const DenseF32Args& g, bool big, hipStream_t st) {
  if (big) return g.bias ? launch_gemm_f32<128, true, AT, BT>(g, st) : launch_gemm_f32<128, false, AT, BT>(g, st);
  return g.bias ? launch_gemm_f32<64, true, AT, BT>(g, st) : launch_gemm_f32<64, false, AT, BT>(g, st);
}

}  // namespace

bool dense_f32_ok(long M, long N, long K, bool at, long lda, bool bt, long ldb, long ldc, const void* a,
                  const void* b, const void* c) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 4 || lda % 4 || ldb % 4) return false;
  if ((at && (M % 4 || lda < M)) || (bt && (N % 4 || ldb < N)) || (!at && lda < K) || (!bt && ldb < K)) return false;
  if (((uintptr_t)a & 15) || ((uintptr_t)b & 15) || ((uintptr_t)c & 3)) return false;
  return fits_f((at ? K : M) * lda * 4) && fits_f((bt ? K : N) * ldb * 4) && fits_f(M * ldc * 4);
}

int dense_f32_gemm(const void* a, int lda, bool at, const void* b, int ldb, bool bt, void* c, int ldc, int M,
                   int N, int K, const void* bias, hipStream_t st) {
  DenseF32Args g{};
  g.a = (const float*)a;
  g.b = (const float*)b;
  g.c = (float*)c;
  g.bias = (const float*)bias;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  g.a_bytes = (int)((long)(at ? K : M) * lda * 4);
  g.b_bytes = (int)((long)(bt ? K : N) * ldb * 4);
  g.c_bytes = (int)((long)M * ldc * 4);
  const bool big = (long)((M + 127) / 128) * ((N + 127) / 128) >= 512;
  if (at) return bt ? launch_layout_f32<true, true>(g, big, st) : launch_layout_f32<true, false>(g, big, st);
  return bt ? launch_layout_f32<false, true>(g, big, st) : launch_layout_f32<false, false>(g, big, st);
}

}  // namespace vh
