// vh_dense.hip -- dense bf16 matrix products (matmul, its gradients, Linear) on
// gfx950 MFMA (v_mfma_f32_32x32x16_bf16), fp32 accumulation.
//
// One kernel form, "NT": C[M][N] = A[M][K] . B[N][K]^T, both operands with the
// contraction index K contiguous (row-major, leading dimensions lda / ldb), so
// every operand tile is a plain copy of 16-byte units into LDS and every MFMA
// fragment (8 consecutive k of one row) is one ds_read_b128.  Products whose
// operands run the other way (matmul's B, the weight gradient's A and G) are
// first transposed into a workspace by transpose_bf16_kernel (tiled through
// LDS: both sides coalesced); that pass moves each operand once, a few percent
// of the product's time at the configs' sizes.
//
// Block: 256 threads (2 x 2 waves), tile BM x BN, K in stages of 64; two LDS
// stages and two register sets: the loads of stage k+2 are issued before the
// MFMAs of stage k (kept there by sched_barrier), the stores of stage k+1 into
// LDS follow them.  XCD-aware block order: the blocks resident on one XCD
// cover groups of 8 m-tiles x a few n-tiles, sharing A and B slices in L2.
#include <type_traits>

#include "vh_kernels.hpp"

namespace vh {

typedef unsigned int u32x4d __attribute__((ext_vector_type(4)));

namespace {

constexpr int kOOR = (int)0x80000000u;  // buffer offset past every range: loads 0, stores dropped
#ifndef VH_GEMM_GROUP_M
#define VH_GEMM_GROUP_M 8
#endif
constexpr int kGroupM = VH_GEMM_GROUP_M;  // m-tiles per group of the block order

struct DenseArgs {
  const uint16_t* a;     // [M][lda]
  const uint16_t* b;     // [N][ldb]
  uint16_t* c;           // [M][ldc]
  const uint16_t* bias;  // [N] or nullptr (added to every row)
  int M, N, K, lda, ldb, ldc;
  int a_bytes, b_bytes, c_bytes;
  int tiles_m, tiles_n;
};

template <int BM, int BN>
struct DenseCfg {
  static constexpr int BK = 64;            // contraction elements per stage
  static constexpr int KU = BK / 8;        // 16-byte units per row per stage
  static constexpr int PU = KU + 1;        // LDS row pitch in units (odd: conflict-free)
  static constexpr int FM = BM / 64, FN = BN / 64;  // 32x32 tiles per wave (waves 2 x 2)
  static constexpr int AIT = BM * KU / 256, BIT = BN * KU / 256;  // load units per thread
  static constexpr int STAGE = (BM + BN) * PU;                     // units per LDS stage
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, bytes, 0x00020000);
}

// PC: 512 threads; waves 0-3 only multiply (consumers, the accumulators),
// waves 4-7 only load the next stages into registers and store them into the
// other LDS buffer (producers, threads 256-511 serving the load map of threads
// 0-255).  Neither role holds the other's registers, so two waves run per SIMD
// and the loads leave the multiplying waves' instruction stream.
template <int BM, int BN, bool BIAS, bool PC = false>
__global__ __launch_bounds__(PC ? 512 : 256)
void gemm_nt_bf16_kernel(DenseArgs g) {
  using Cfg = DenseCfg<BM, BN>;
  constexpr int FM = Cfg::FM, FN = Cfg::FN, PU = Cfg::PU, STAGE = Cfg::STAGE;
  extern __shared__ __attribute__((aligned(16))) u32x4d lds[];
  const bool producer = PC && threadIdx.x >= 256;
  const int tid = PC ? (int)(threadIdx.x & 255u) : (int)threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);
  // logical block -> tile in groups of up to 8 m-tiles: consecutive logical
  // blocks (the ones resident on one XCD at a time) walk 8 m-tiles, then the
  // next n-tile, so they share both A and B slices in that XCD's L2 (32 of them
  // cover 8 x 4 tiles instead of 1 x 32)
  const int lb = xcd_block(g.tiles_m * g.tiles_n);
  const int grp = lb / (kGroupM * g.tiles_n), first_m = grp * kGroupM;
  const int gm = min(g.tiles_m - first_m, kGroupM);
  const int in_grp = lb - grp * kGroupM * g.tiles_n;
  const int m0 = (first_m + in_grp % gm) * BM, n0 = (in_grp / gm) * BN;

  // load items: unit u = tid + 256*it -> row u / KU, column unit u % KU (= tid % KU)
  const int cu = tid % Cfg::KU;
  int a_off[Cfg::AIT], b_off[Cfg::BIT];
#pragma unroll
  for (int it = 0; it < Cfg::AIT; ++it) {
    const int r = (tid + it * 256) / Cfg::KU;
    a_off[it] = m0 + r < g.M ? ((m0 + r) * g.lda + cu * 8) * 2 : kOOR;
  }
#pragma unroll
  for (int it = 0; it < Cfg::BIT; ++it) {
    const int r = (tid + it * 256) / Cfg::KU;
    b_off[it] = n0 + r < g.N ? ((n0 + r) * g.ldb + cu * 8) * 2 : kOOR;
  }
  const __amdgpu_buffer_rsrc_t ar = rsrc(g.a, g.a_bytes), br = rsrc(g.b, g.b_bytes);

  u32x4d areg[2][Cfg::AIT], breg[2][Cfg::BIT];
  auto gload = [&](auto SET, int k0) {
    constexpr int s = decltype(SET)::value;
    const bool kin = k0 + cu * 8 < g.K;  // K % 8 == 0: a unit is all in or all out
#pragma unroll
    for (int it = 0; it < Cfg::AIT; ++it)
      areg[s][it] = __builtin_bit_cast(u32x4d,
                                       __builtin_amdgcn_raw_buffer_load_b128(ar, kin ? a_off[it] : kOOR, k0 * 2, 0));
#pragma unroll
    for (int it = 0; it < Cfg::BIT; ++it)
      breg[s][it] = __builtin_bit_cast(u32x4d,
                                       __builtin_amdgcn_raw_buffer_load_b128(br, kin ? b_off[it] : kOOR, k0 * 2, 0));
  };
  auto sstore = [&](auto SET, int st) {
    constexpr int s = decltype(SET)::value;
    u32x4d* base = lds + st * STAGE;
#pragma unroll
    for (int it = 0; it < Cfg::AIT; ++it) base[((tid + it * 256) / Cfg::KU) * PU + cu] = areg[s][it];
#pragma unroll
    for (int it = 0; it < Cfg::BIT; ++it) base[(BM + (tid + it * 256) / Cfg::KU) * PU + cu] = breg[s][it];
  };

  f32x16 acc[FM][FN];
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};
  };
  if (!PC) zero_acc();
  const int row_l = lane & 31, half_l = lane >> 5;
  auto compute = [&](int st) {
    const u32x4d* ap = lds + st * STAGE + (wm + row_l) * PU + half_l;
    const u32x4d* bp = lds + st * STAGE + (BM + wn + row_l) * PU + half_l;
#pragma unroll
    for (int ks = 0; ks < Cfg::KU; ks += 2) {
      bf16x8 af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) af[i] = __builtin_bit_cast(bf16x8, ap[i * 32 * PU + ks]);
#pragma unroll
      for (int j = 0; j < FN; ++j) bf[j] = __builtin_bit_cast(bf16x8, bp[j * 32 * PU + ks]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  const int nk = (g.K + Cfg::BK - 1) / Cfg::BK;
  if constexpr (PC) {
    // one barrier per stage on both sides; stage k is multiplied from buffer
    // k & 1 while the producers store stage k+1 into the other buffer (read
    // by the consumers before the previous barrier) and load stage k+3
    if (producer) {
      gload(I0{}, 0);
      if (nk > 1) gload(I1{}, Cfg::BK);
      __builtin_amdgcn_sched_barrier(0);
      sstore(I0{}, 0);
      if (nk > 2) gload(I0{}, 2 * Cfg::BK);
      __syncthreads();
      for (int kt = 0; kt < nk; kt += 2) {
        if (kt + 1 < nk) sstore(I1{}, 1);
        if (kt + 3 < nk) gload(I1{}, (kt + 3) * Cfg::BK);
        __syncthreads();
        if (kt + 1 >= nk) break;
        if (kt + 2 < nk) sstore(I0{}, 0);
        if (kt + 4 < nk) gload(I0{}, (kt + 4) * Cfg::BK);
        __syncthreads();
      }
      return;
    }
    zero_acc();
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      compute(kt & 1);
      __syncthreads();
    }
  } else {
  // invariant at an even stage k: LDS buffer 0 holds stage k, register set 1
  // holds stage k+1 (in flight), set 0 is free
  gload(I0{}, 0);
  if (nk > 1) gload(I1{}, Cfg::BK);
  __builtin_amdgcn_sched_barrier(0);
  sstore(I0{}, 0);
  __syncthreads();
  int kt = 0;
  for (; kt + 3 < nk; kt += 2) {
    gload(I0{}, (kt + 2) * Cfg::BK);
    __builtin_amdgcn_sched_barrier(0);
    compute(0);
    __builtin_amdgcn_sched_barrier(0);
    sstore(I1{}, 1);
    __syncthreads();
    gload(I1{}, (kt + 3) * Cfg::BK);
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
    __builtin_amdgcn_sched_barrier(0);
    sstore(I0{}, 0);
    __syncthreads();
  }
  const int rem = nk - kt;  // 1, 2 or 3 stages left
  if (rem == 3) gload(I0{}, (kt + 2) * Cfg::BK);
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
  }

  // epilogue: fp32 (+ bias), one rounding, row-major stores (lanes walk columns)
  const __amdgpu_buffer_rsrc_t cr = rsrc(g.c, g.c_bytes);
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int col = n0 + wn + j * 32 + row_l;
    const bool cok = col < g.N;
    const float bv = (BIAS && cok) ? bf16_to_f32(g.bias[col]) : 0.f;
    const int voff = cok ? (col + half_l * 4 * g.ldc) * 2 : kOOR;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm + i * 32 + (v >> 2) * 8 + (v & 3);  // + 4 * half_l
        if (row + half_l * 4 < g.M)
          __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (__bf16)(acc[i][j][v] + bv)), cr,
                                                voff, row * g.ldc * 2, 0);
      }
  }
}

// out[c][r] = in[r][c] for a bf16 [R][Cc] matrix (leading dimension ldi) into a
// dense [Cc][R] one.  64 x 64 tiles: 16-byte loads along rows, the transposed
// tile in LDS, 16-byte stores along the output rows.  R % 8 == 0, Cc % 8 == 0.
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const uint16_t* __restrict__ in, int ldi,
                                                             uint16_t* __restrict__ out, int R, int Cc) {
  __shared__ uint16_t t[64][64 + 8];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int u = tid + k * 256;  // 512 units of 8 elements: row u / 8, column unit u % 8
    const int r = u >> 3, cu = u & 7;
    if (r0 + r < R && c0 + cu * 8 < Cc) {
      const u32x4d v = *reinterpret_cast<const u32x4d*>(in + (size_t)(r0 + r) * ldi + c0 + cu * 8);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        t[cu * 8 + 2 * e][r] = (uint16_t)(v[e] & 0xffffu);
        t[cu * 8 + 2 * e + 1][r] = (uint16_t)(v[e] >> 16);
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int u = tid + k * 256;  // output row (input column) u / 8, unit u % 8
    const int c = u >> 3, ru = u & 7;
    if (c0 + c < Cc && r0 + ru * 8 < R)
      *reinterpret_cast<u32x4d*>(out + (size_t)(c0 + c) * R + r0 + ru * 8) =
          *reinterpret_cast<const u32x4d*>(&t[c][ru * 8]);
  }
}

bool fits(long bytes) { return bytes >= 0 && bytes < (1L << 31) - 64; }

template <int BM, int BN, bool BIAS, bool PC = false>
int launch_nt(const DenseArgs& a0, hipStream_t st) {
  using Cfg = DenseCfg<BM, BN>;
  auto kern = gemm_nt_bf16_kernel<BM, BN, BIAS, PC>;
  const size_t lds = (size_t)2 * Cfg::STAGE * 16;
  VH_LDS_LIMIT_ONCE(kern);
  DenseArgs a = a0;
  a.tiles_m = (a.M + BM - 1) / BM;
  a.tiles_n = (a.N + BN - 1) / BN;
  kern<<<dim3((unsigned)(a.tiles_m * a.tiles_n)), PC ? 512 : 256, lds, st>>>(a);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

}  // namespace

bool dense_nt_bf16_ok(long M, long N, long K, long lda, long ldb, long ldc, const void* a, const void* b,
                      const void* c) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 8 || lda % 8 || ldb % 8) return false;
  if (((uintptr_t)a & 15) || ((uintptr_t)b & 15) || ((uintptr_t)c & 1)) return false;
  return fits(M * lda * 2) && fits(N * ldb * 2) && fits(M * ldc * 2);
}

int dense_nt_bf16(const void* a, int lda, const void* b, int ldb, void* c, int ldc, int M, int N, int K,
                  const void* bias, hipStream_t st) {
  DenseArgs g{};
  g.a = (const uint16_t*)a;
  g.b = (const uint16_t*)b;
  g.c = (uint16_t*)c;
  g.bias = (const uint16_t*)bias;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  g.a_bytes = (int)((long)M * lda * 2);
  g.b_bytes = (int)((long)N * ldb * 2);
  g.c_bytes = (int)((long)M * ldc * 2);
  // 128 x 256 tiles (one block per CU, producer / consumer form, 64 x 128 per
  // consumer wave) when the grid still fills the chip, else 128 x 128 (two
  // blocks per CU of four waves that both load and multiply: already two waves
  // per SIMD, and measured as fast as or faster than a split form)
  const long big = (long)((M + 127) / 128) * ((N + 255) / 256);
  if (big >= 256) return bias ? launch_nt<128, 256, true, true>(g, st) : launch_nt<128, 256, false, true>(g, st);
  return bias ? launch_nt<128, 128, true>(g, st) : launch_nt<128, 128, false>(g, st);
}

int transpose_bf16(const void* in, int ldi, void* out, int R, int Cc, hipStream_t st) {
  if (R % 8 || Cc % 8) return set_error(VH_ERR_UNSUPPORTED, "transpose needs multiples of 8");
  dim3 grid((unsigned)((Cc + 63) / 64), (unsigned)((R + 63) / 64));
  transpose_bf16_kernel<<<grid, 256, 0, st>>>((const uint16_t*)in, ldi, (uint16_t*)out, R, Cc);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

}  // namespace vh
