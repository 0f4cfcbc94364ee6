// vh_dense.hip -- dense bf16 matrix products (matmul, its gradients, Linear) on
// gfx950 MFMA (v_mfma_f32_32x32x16_bf16), fp32 accumulation.
//
// One kernel for C[M][N] = A . B with either operand stored either way:
// "K-major" (row-major [rows][K], the contraction index contiguous: A[M][K],
// B[N][K]) or "MN-major" ([K][rows], the row index contiguous: A stored
// [K][M], B stored [K][N] -- matmul's B, the weight gradient's A and G).  Every
// operand tile is a plain copy of 16-byte units into LDS in its stored order.
// An MFMA fragment (8 consecutive k of one row) of a K-major tile is one
// ds_read_b128; of an MN-major tile ([k][row] in LDS) it is two
// ds_read_b64_tr_b16, gfx950's transposing LDS read: within each group of 16
// lanes, lane i names 4 consecutive elements of row i/4 (elements
// 4*(i%4) .. +3), and lane j receives element j of each of the 4 rows, i.e. 4
// consecutive k of column j.  No operand is transposed in memory.
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
typedef unsigned int u32x2d __attribute__((ext_vector_type(2)));

namespace {

constexpr int kOOR = (int)0x80000000u;  // buffer offset past every range: loads 0, stores dropped
#ifndef VH_GEMM_GROUP_M
#define VH_GEMM_GROUP_M 8
#endif
constexpr int kGroupM = VH_GEMM_GROUP_M;  // m-tiles per group of the block order

struct DenseArgs {
  const uint16_t* a;     // [M][lda] (K-major) or [K][lda] (MN-major)
  const uint16_t* b;     // [N][ldb] (K-major) or [K][ldb] (MN-major)
  uint16_t* c;           // [M][ldc]
  const uint16_t* bias;  // [N] or nullptr (added to every row)
  uint16_t* colsum;      // [N] or nullptr: column sums of an MN-major B over K (128 x 128 tiles only)
  int cs_shift;          // columns per block of the column sums: 4 << cs_shift (set at launch)
  int vec_epi;           // C 16-byte aligned, ldc and N multiples of 8: 16-byte stores through LDS
  int M, N, K, lda, ldb, ldc;
  int a_bytes, b_bytes, c_bytes;
  int tiles_m, tiles_n;
};

template <int BM, int BN, bool AT = false, bool BT = false>
struct DenseCfg {
  static constexpr int BK = 64;            // contraction elements per stage
  static constexpr int KU = BK / 8;        // 16-byte units per row per stage
  static constexpr int PU = KU + 1;        // K-major tile: LDS row pitch in units (odd: conflict-free)
  static constexpr int FM = BM / 64, FN = BN / 64;  // 32x32 tiles per wave (waves 2 x 2)
  static constexpr int AIT = BM * KU / 256, BIT = BN * KU / 256;  // load units per thread
  // MN-major tile: BK rows of R elements, pitch R + 32 elements (row starts 64
  // bytes apart mod 256: the four rows of a transposing read hit disjoint banks)
  static constexpr int mn_pitch(int R) { return R / 8 + 4; }
  static constexpr int A_UNITS = AT ? BK * mn_pitch(BM) : BM * PU;
  static constexpr int B_UNITS = BT ? BK * mn_pitch(BN) : BN * PU;
  static constexpr int STAGE = A_UNITS + B_UNITS;  // units per LDS stage
  // producer / consumer tiles with an MN-major B: room after the two stages
  // for the producers' column-sum exchange (256 / (BN / 8) k-row groups x at
  // most BN columns, fp32)
  static constexpr int CS_BYTES = BT ? 256 / (BN / 8) * BN * 4 : 0;
  static constexpr size_t lds_bytes(bool pc) { return (size_t)2 * STAGE * 16 + (pc ? CS_BYTES : 0); }
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, bytes, 0x00020000);
}

// PC: 512 threads; waves 0-3 only multiply (consumers, the accumulators),
// waves 4-7 only load the next stages into registers and store them into the
// other LDS buffer (producers, threads 256-511 serving the load map of threads
// 0-255).  Neither role holds the other's registers, so two waves run per SIMD
// and the loads leave the multiplying waves' instruction stream.
// One block's tile: logical block lb of the grid order below.
template <int BM, int BN, bool BIAS, bool PC, bool AT, bool BT>
__device__ __forceinline__ void gemm_bf16_tile(const DenseArgs& g, const int lb) {
  using Cfg = DenseCfg<BM, BN, AT, BT>;
  constexpr int FM = Cfg::FM, FN = Cfg::FN, PU = Cfg::PU, STAGE = Cfg::STAGE;
  constexpr int APU = Cfg::mn_pitch(BM), BPU = Cfg::mn_pitch(BN);  // MN-major LDS pitches (units)
  extern __shared__ __attribute__((aligned(16))) u32x4d lds[];
  const bool producer = PC && threadIdx.x >= 256;
  const int tid = PC ? (int)(threadIdx.x & 255u) : (int)threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);
  // logical block -> tile in groups of up to 8 m-tiles: consecutive logical
  // blocks (the ones resident on one XCD at a time) walk 8 m-tiles, then the
  // next n-tile, so they share both A and B slices in that XCD's L2 (32 of them
  // cover 8 x 4 tiles instead of 1 x 32)
  const int grp = lb / (kGroupM * g.tiles_n), first_m = grp * kGroupM;
  const int gm = min(g.tiles_m - first_m, kGroupM);
  const int in_grp = lb - grp * kGroupM * g.tiles_n;
  const int m0 = (first_m + in_grp % gm) * BM, n0 = (in_grp / gm) * BN;

  // Load items.  K-major operand: unit u = tid + 256*it -> row u / KU, k unit
  // u % KU (= tid % KU); global offset of k0 = 0 (the stage's k0 is a scalar
  // offset).  MN-major operand: unit u -> k row u / (R/8), row unit u % (R/8);
  // the k row's bound is checked per unit (a scalar offset is not range-checked,
  // so an unused unit carries an out-of-range per-lane offset).
  const int cu = tid % Cfg::KU;
  int a_off[Cfg::AIT], b_off[Cfg::BIT], a_kr[Cfg::AIT], b_kr[Cfg::BIT], a_l[Cfg::AIT], b_l[Cfg::BIT];
#pragma unroll
  for (int it = 0; it < Cfg::AIT; ++it) {
    const int u = tid + it * 256;
    if constexpr (AT) {
      const int kr = u / (BM / 8), ru = u % (BM / 8);
      a_kr[it] = kr;
      a_off[it] = m0 + ru * 8 < g.M ? (kr * g.lda + m0 + ru * 8) * 2 : kOOR;
      a_l[it] = kr * APU + ru;
    } else {
      const int r = u / Cfg::KU;
      a_kr[it] = cu * 8;
      a_off[it] = m0 + r < g.M ? ((m0 + r) * g.lda + cu * 8) * 2 : kOOR;
      a_l[it] = r * PU + cu;
    }
  }
#pragma unroll
  for (int it = 0; it < Cfg::BIT; ++it) {
    const int u = tid + it * 256;
    if constexpr (BT) {
      const int kr = u / (BN / 8), ru = u % (BN / 8);
      b_kr[it] = kr;
      b_off[it] = n0 + ru * 8 < g.N ? (kr * g.ldb + n0 + ru * 8) * 2 : kOOR;
      b_l[it] = Cfg::A_UNITS + kr * BPU + ru;
    } else {
      const int r = u / Cfg::KU;
      b_kr[it] = cu * 8;
      b_off[it] = n0 + r < g.N ? ((n0 + r) * g.ldb + cu * 8) * 2 : kOOR;
      b_l[it] = Cfg::A_UNITS + r * PU + cu;
    }
  }
  const __amdgpu_buffer_rsrc_t ar = rsrc(g.a, g.a_bytes), br = rsrc(g.b, g.b_bytes);

  u32x4d areg[2][Cfg::AIT], breg[2][Cfg::BIT];
  auto gload = [&](auto SET, int k0) {
    constexpr int s = decltype(SET)::value;
    // k0 as a scalar offset: k0 elements along a K-major row, k0 rows of an MN-major operand
    const int ask = AT ? k0 * g.lda * 2 : k0 * 2, bsk = BT ? k0 * g.ldb * 2 : k0 * 2;
#pragma unroll
    for (int it = 0; it < Cfg::AIT; ++it)  // K % 8 == 0: a K-major unit is all in or all out
      areg[s][it] = __builtin_bit_cast(
          u32x4d, __builtin_amdgcn_raw_buffer_load_b128(ar, k0 + a_kr[it] < g.K ? a_off[it] : kOOR, ask, 0));
#pragma unroll
    for (int it = 0; it < Cfg::BIT; ++it)
      breg[s][it] = __builtin_bit_cast(
          u32x4d, __builtin_amdgcn_raw_buffer_load_b128(br, k0 + b_kr[it] < g.K ? b_off[it] : kOOR, bsk, 0));
  };
  // Column sums of B over K (a Linear weight gradient's bias gradient, B = dY
  // stored [K][N]).  The tiling's tiles_m blocks of a column tile each own
  // 4 << cs_shift of its columns (block of m-tile mt: columns mt * width ..
  // + width - 1), so every column is summed by exactly one block, over all K.
  //  * 4-wave blocks: from the staged LDS tile -- a thread adds 4 consecutive
  //    owned columns of the k rows tid >> cs_shift (+ 256 >> cs_shift ...) of
  //    each stage, in stage order; the thread sums are added in k-row order.
  //  * producer / consumer blocks: the producers add the owned B units they
  //    hold in registers before storing them (a thread's units all cover the
  //    same 8 columns: unit tid + 256 it has row unit tid % (BN / 8)), stage by
  //    stage; the 256 / (BN / 8) k-row group sums are added in group order.
  constexpr bool CS = BT;
  constexpr int RU = BN / 8;  // row units per k row of the B tile
  static_assert(256 % RU == 0, "a thread's B units must share their columns");
  const int cs_w = 4 << g.cs_shift, cs_c0 = (m0 / BM) * cs_w;
  const bool cs_on = CS && g.colsum != nullptr;  // block-uniform
  const bool cs_blk = cs_on && cs_c0 < BN;
  const int cs_g = tid & ((1 << g.cs_shift) - 1), cs_k0 = tid >> g.cs_shift;
  const int cs_ru = tid % RU;
  const bool cs_own = cs_blk && cs_ru * 8 >= cs_c0 && cs_ru * 8 < cs_c0 + cs_w;
  float csum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  auto colsum_stage = [&](int st) {
    const char* bt = reinterpret_cast<const char*>(lds + st * STAGE + Cfg::A_UNITS);
    for (int k = cs_k0; k < Cfg::BK; k += 256 >> g.cs_shift) {
      const u32x2d v = *reinterpret_cast<const u32x2d*>(bt + k * BPU * 16 + (cs_c0 + cs_g * 4) * 2);
      csum[0] += __builtin_bit_cast(float, v[0] << 16);
      csum[1] += __builtin_bit_cast(float, v[0] & 0xffff0000u);
      csum[2] += __builtin_bit_cast(float, v[1] << 16);
      csum[3] += __builtin_bit_cast(float, v[1] & 0xffff0000u);
    }
  };
  auto sstore = [&](auto SET, int st) {
    constexpr int s = decltype(SET)::value;
    u32x4d* base = lds + st * STAGE;
#pragma unroll
    for (int it = 0; it < Cfg::AIT; ++it) base[a_l[it]] = areg[s][it];
#pragma unroll
    for (int it = 0; it < Cfg::BIT; ++it) base[b_l[it]] = breg[s][it];
    if constexpr (CS && PC) {
      if (cs_own) {
#pragma unroll
        for (int it = 0; it < Cfg::BIT; ++it)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const unsigned w = breg[s][it][e];
            csum[2 * e] += __builtin_bit_cast(float, w << 16);
            csum[2 * e + 1] += __builtin_bit_cast(float, w & 0xffff0000u);
          }
      }
    }
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
  // transposing reads of an MN-major tile: lane l reads k row 8*(l/32) + (l%16)/4
  // (+4 for the second half of the fragment), elements 16*((l/16)%2) + 4*(l%4) .. +3
  const int tr_row = 8 * half_l + ((lane & 15) >> 2), tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  auto frag_mn = [&](const u32x4d* tile, int pitch_units, int ks, int col0) {
    typedef short v4i16 __attribute__((ext_vector_type(4)));
    const __attribute__((address_space(3))) char* p =
        (const __attribute__((address_space(3))) char*)(tile) +
        (((ks * 8 + tr_row) * pitch_units) * 16 + (col0 + tr_col) * 2);
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)p);
    const v4i16 hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)(p + 4 * pitch_units * 16));
    typedef short v8i16 __attribute__((ext_vector_type(8)));
    const v8i16 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8, v);
  };
  auto compute = [&](int st) {
    const u32x4d* ap = lds + st * STAGE + (wm + row_l) * PU + half_l;
    const u32x4d* bp = lds + st * STAGE + Cfg::A_UNITS + (wn + row_l) * PU + half_l;
    const u32x4d* at = lds + st * STAGE;
    const u32x4d* bt = lds + st * STAGE + Cfg::A_UNITS;
#pragma unroll
    for (int ks = 0; ks < Cfg::KU; ks += 2) {
      bf16x8 af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = AT ? frag_mn(at, APU, ks, wm + i * 32) : __builtin_bit_cast(bf16x8, ap[i * 32 * PU + ks]);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[j] = BT ? frag_mn(bt, BPU, ks, wn + j * 32) : __builtin_bit_cast(bf16x8, bp[j * 32 * PU + ks]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if constexpr (CS && !PC) {  // after the stage's MFMAs are issued: the adds overlap their execution
      if (cs_blk) colsum_stage(st);
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
      if constexpr (CS) {
        if (cs_on) {
          float* red = reinterpret_cast<float*>(lds + 2 * STAGE);  // [256 / RU][cs_w]
          if (cs_own) {
#pragma unroll
            for (int e = 0; e < 8; ++e) red[(tid / RU) * cs_w + cs_ru * 8 - cs_c0 + e] = csum[e];
          }
          __syncthreads();  // matched by the consumers after their last stage
          const int n = n0 + cs_c0 + tid;
          if (cs_blk && tid < cs_w && n < g.N) {
            float t = 0.f;
            for (int j = 0; j < 256 / RU; ++j) t += red[j * cs_w + tid];
            g.colsum[n] = f32_to_bf16(t);
          }
        }
      }
      return;
    }
    zero_acc();
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      compute(kt & 1);
      __syncthreads();
    }
    if constexpr (CS) {
      if (cs_on) __syncthreads();  // the producers' column-sum exchange
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

  if constexpr (CS && !PC) {
    if (cs_blk) {  // per owned column: the 256 >> cs_shift k-row sums, added in k-row order
      static_assert(256 * 4 * 4 <= 2 * STAGE * 16, "column-sum exchange exceeds the LDS stages");
      __syncthreads();  // every wave is done reading the last stage
      float* red = reinterpret_cast<float*>(lds);
#pragma unroll
      for (int e = 0; e < 4; ++e) red[cs_k0 * cs_w + cs_g * 4 + e] = csum[e];
      __syncthreads();
      const int n = n0 + cs_c0 + tid;
      if (tid < cs_w && n < g.N) {
        float t = 0.f;
        for (int j = 0; j < 256 >> g.cs_shift; ++j) t += red[j * cs_w + tid];
        g.colsum[n] = f32_to_bf16(t);
      }
    }
  }

  const __amdgpu_buffer_rsrc_t cr = rsrc(g.c, g.c_bytes);
  if (g.vec_epi) {
    // epilogue: fp32 (+ bias), one rounding, the wave's tile through its own LDS
    // region (pitch WN + 8 elements), then out as 16-byte runs of 8 columns: 16
    // (8) stores per lane instead of 128 (64) two-byte ones
    constexpr int WMR = FM * 32, WN = FN * 32, EP = WN + 8, CPR = WN / 8, RPI = 64 / CPR;
    static_assert(4 * WMR * EP * 2 <= 2 * STAGE * 16, "epilogue tiles exceed the LDS stages");
    if constexpr (!PC) __syncthreads();  // PC: the consumers' last stage barrier already passed
    uint16_t* eb = reinterpret_cast<uint16_t*>(lds) + wave * WMR * EP;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int cw = j * 32 + row_l, col = n0 + wn + cw;
      const float bv = (BIAS && col < g.N) ? bf16_to_f32(g.bias[col]) : 0.f;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          eb[(i * 32 + (v >> 2) * 8 + half_l * 4 + (v & 3)) * EP + cw] =
              __builtin_bit_cast(uint16_t, (__bf16)(acc[i][j][v] + bv));
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
    const int ch = lane % CPR, col = n0 + wn + ch * 8;
#pragma unroll
    for (int it = 0; it < WMR / RPI; ++it) {
      const int rw = it * RPI + lane / CPR, row = m0 + wm + rw;
      const u32x4d v = *reinterpret_cast<const u32x4d*>(eb + rw * EP + ch * 8);
      __builtin_amdgcn_raw_buffer_store_b128(v, cr, row < g.M && col < g.N ? (row * g.ldc + col) * 2 : kOOR, 0, 0);
    }
    return;
  }
  // epilogue: fp32 (+ bias), one rounding, row-major stores (lanes walk columns)
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

template <int BM, int BN, bool BIAS, bool PC = false, bool AT = false, bool BT = false>
__global__ __launch_bounds__(PC ? 512 : 256)
void gemm_bf16_kernel(DenseArgs g) {
  gemm_bf16_tile<BM, BN, BIAS, PC, AT, BT>(g, xcd_block(g.tiles_m * g.tiles_n));
}

// Two independent products in one launch: blocks 0 .. T0-1 take the first
// product's tiles, the rest the second's.  Meant for pairs whose grids would
// each leave half the chip idle (a Linear layer's dX and dW): together they
// fill it -- 128 x 256 producer / consumer tiles, one block per CU, when the
// two grids reach a block per CU, else 128 x 128 tiles at two blocks per CU.
template <int BN, bool PC, bool AT0, bool BT0, bool AT1, bool BT1>
__global__ __launch_bounds__(PC ? 512 : 256)
void gemm_bf16_pair_kernel(DenseArgs g0, DenseArgs g1) {
  const int t0 = g0.tiles_m * g0.tiles_n, h = blockIdx.x;
  if (h < t0)
    gemm_bf16_tile<128, BN, false, PC, AT0, BT0>(g0, xcd_map(h, t0));
  else
    gemm_bf16_tile<128, BN, false, PC, AT1, BT1>(g1, xcd_map(h - t0, g1.tiles_m * g1.tiles_n));
}

// ---------------------------------------------------------------- BM x 256 tiles, direct-to-LDS loads
// For products whose tiles are whole (M a multiple of BM, N of 256, K of 128):
// the square product and its gradients and a Linear forward on 256 x 256
// tiles, a Linear layer's dX and dW as one launch on 128 x 256 tiles.  The
// operands are copied from global memory straight into LDS by
// buffer_load_dwordx4 ... lds (no registers and no LDS store instructions on
// the way), two LDS stages of 64 k, the copies of stage s+1 issued when stage
// s starts.  Eight waves split the tile 2 (m) x 4 (n): BM/2 x 64 per wave
// (256 x 256: 128 accumulator registers, two waves per SIMD, so one wave's
// copy issue and barrier waits are covered by the other's MFMAs).  Measured on
// 8192^3 (one box): eight waves 5-15 % faster than four waves of 128 x 128;
// 64-k stages 2-5 % faster than four stages of 32 k (whole 128-byte lines of
// the K-major rows, half the barriers).
// LDS DMA writes a wave's 64 16-byte units contiguously (lane l at unit l of
// the instruction's base), so a tile's layout is set by which global unit each
// lane fetches; an XOR swizzle of the unit index keeps the fragment reads
// free of bank conflicts (16 consecutive lanes on 16 distinct 16-byte bank
// groups; measured: 0.8 % conflict cycles):
//  * K-major tile (R rows x 64 k, 8 units per row, row r at units 8r ..
//    8r+7): slot t of row r holds k unit t ^ ((r >> 1) & 7).  Copy
//    instruction c covers rows 8c .. 8c+7.
//  * MN-major tile (64 k rows x R, UR = R/8 units per k row): slot t of k row
//    kr holds row unit t ^ (4 (kr & 3)).  Instruction c covers 64/UR k rows.
// The copies are issued as inline assembly, so the compiler's wait-count pass
// does not see them (it would otherwise order fragment reads after all copies
// in flight): the waits are explicit -- vmcnt(0) for the thread's own copies
// of the next stage, lgkmcnt(0) for its fragment reads -- in one statement
// with the s_barrier, which clobbers memory so that no LDS read moves across
// it.  The two stages are separate static arrays and the main loop is
// unrolled by two.
constexpr int kD2lBK = 64;  // k per stage

// buffer_load_dwordx4 ... lds: lane l's 16 bytes (voff + soff) land at LDS
// byte la + 16 l; M0 holds la (the s_nop covers the M0 -> LDS DMA hazard).
// M0 is listed as clobbered; nothing else in these kernels uses it (their
// generated code references M0 only in these copies).
__device__ __forceinline__ void d2l_copy(__amdgpu_buffer_rsrc_t r, int voff, int soff, uint32_t la) {
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(r), "s"(soff), "s"(la)
               : "memory", "m0");
}

// s_waitcnt vmcnt(0) lgkmcnt(0), then the block barrier
__device__ __forceinline__ void d2l_sync() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ uint32_t lds_addr(const u32x4d* p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) u32x4d*)p);
}

// Tile geometry: BM x 256 (BM = 256 or 128), eight waves 2 (m) x 4 (n) of
// BM/2 x 64 each, two LDS stages of (BM + 256) x 64 bf16.
template <int BM>
struct D2lCfg {
  static constexpr int FM = BM / 64, FN = 2;             // 32 x 32 fragments per wave
  static constexpr int A_UNITS = BM * 8, B_UNITS = 2048;  // 16-byte units per stage
  static constexpr int STAGE = A_UNITS + B_UNITS;
  static constexpr int ACPW = BM / 64, BCPW = 4;          // copy instructions per wave and stage
};

// One BM x 256 tile of C = A . B (logical block lb), S0 / S1 the two stages.
// CS: the column sums of an MN-major B over K (a Linear weight gradient's bias
// gradient) from the staged tiles: the tiles_m blocks of a column tile each
// own 4 << cs_shift of its columns (block of m-tile mt: columns mt * width ..),
// so every column is summed by exactly one block, over all K; a thread adds 4
// consecutive owned columns of one k row per stage, in stage order, and the
// k-row group sums are added in group order at the end.
template <int BM, bool AT, bool BT, bool BIAS, bool CS>
__device__ __forceinline__ void d2l_tile(const DenseArgs& g, const int lb, u32x4d* S0, u32x4d* S1) {
  using Cfg = D2lCfg<BM>;
  constexpr int FM = Cfg::FM, FN = Cfg::FN, UNITS_A = Cfg::A_UNITS;
  constexpr int BKX = kD2lBK;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave >> 2) * (BM / 2), wn = (wave & 3) * 64;
  const int grp = lb / (kGroupM * g.tiles_n), first_m = grp * kGroupM;
  const int gm = min(g.tiles_m - first_m, kGroupM);
  const int in_grp = lb - grp * kGroupM * g.tiles_n;
  const int m0 = (first_m + in_grp % gm) * BM, n0 = (in_grp / gm) * 256;

  // copy instruction c of an operand with R rows (R = BM or 256):
  //  K-major: rows 8c .. 8c+7, lane -> row 8c + lane/8, slot lane%8 holds k
  //    unit (lane%8) ^ ((row >> 1) & 7);
  //  MN-major (UR = R/8 units per k row): k rows (64/UR) c .. , lane -> k row
  //    (64/UR) c + lane/UR, slot lane%UR holds row unit slot ^ (4 (kr & 3)).
  auto unit_off = [&](bool mn, int R, int rc0, int ld, int c) {
    if (!mn) {
      const int r = 8 * c + (lane >> 3), u = (lane & 7) ^ ((r >> 1) & 7);
      return ((rc0 + r) * ld + 8 * u) * 2;
    }
    const int UR = R / 8;
    const int kr = (64 / UR) * c + lane / UR, mu = (lane % UR) ^ (4 * (kr & 3));
    return (kr * ld + rc0 + 8 * mu) * 2;
  };
  int aoff[Cfg::ACPW], boff[Cfg::BCPW];
#pragma unroll
  for (int i = 0; i < Cfg::ACPW; ++i) aoff[i] = unit_off(AT, BM, m0, g.lda, Cfg::ACPW * wave + i);
#pragma unroll
  for (int i = 0; i < Cfg::BCPW; ++i) boff[i] = unit_off(BT, 256, n0, g.ldb, Cfg::BCPW * wave + i);
  const __amdgpu_buffer_rsrc_t ar = rsrc(g.a, g.a_bytes), br = rsrc(g.b, g.b_bytes);
  auto issue = [&](u32x4d* st, int k0) {
    const int ask = __builtin_amdgcn_readfirstlane(AT ? k0 * g.lda * 2 : k0 * 2);
    const int bsk = __builtin_amdgcn_readfirstlane(BT ? k0 * g.ldb * 2 : k0 * 2);
    const uint32_t la = lds_addr(st);
#pragma unroll
    for (int i = 0; i < Cfg::ACPW; ++i) d2l_copy(ar, aoff[i], ask, la + (Cfg::ACPW * wave + i) * 64 * 16);
#pragma unroll
    for (int i = 0; i < Cfg::BCPW; ++i)
      d2l_copy(br, boff[i], bsk, la + (UNITS_A + (Cfg::BCPW * wave + i) * 64) * 16);
  };

  // fragment addresses (bytes from the operand tile's start) of k step kk (0 .. 3)
  const int row_l = lane & 31, half_l = lane >> 5;
  // K-major: row = base + row_l (base a multiple of 32), k unit 2 kk + half_l
  int kfrag[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) kfrag[kk] = (8 * row_l + ((2 * kk + half_l) ^ ((row_l >> 1) & 7))) * 16;
  // MN-major (transposing reads, UR units per k row): k row 16 kk + 8 half_l +
  // (lane & 15) / 4 (+4 for the second read), columns 16 ((lane >> 4) & 1) +
  // 4 (lane & 3) .. +3
  const int tr_row = 8 * half_l + ((lane & 15) >> 2), x4 = 4 * ((lane >> 2) & 3);
  const int tr_in = (2 * ((lane >> 4) & 1) + ((lane & 3) >> 1)) * 16 + 8 * (lane & 1);
  auto mn_frag = [&](int UR, int col0) { return tr_row * UR * 16 + tr_in + ((col0 >> 3) ^ x4) * 16; };
  int amn[FM], bmn[FN];
#pragma unroll
  for (int f = 0; f < FM; ++f) amn[f] = mn_frag(BM / 8, wm + 32 * f);
#pragma unroll
  for (int f = 0; f < FN; ++f) bmn[f] = mn_frag(32, wn + 32 * f);
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef short v8i16 __attribute__((ext_vector_type(8)));
  auto read_tr = [&](const u32x4d* tile, int byte, int UR) {
    const __attribute__((address_space(3))) char* p = (const __attribute__((address_space(3))) char*)tile + byte;
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)p);
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)(p + 4 * UR * 16));
    const v8i16 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8, v);
  };
  struct Frags {
    bf16x8 a[FM], b[FN];
  };
  auto read = [&](const u32x4d* st, int kk, Frags& f) {
    const u32x4d* at = st;
    const u32x4d* bt = st + UNITS_A;
#pragma unroll
    for (int i = 0; i < FM; ++i)
      f.a[i] = AT ? read_tr(at, amn[i] + kk * 16 * (BM / 8) * 16, BM / 8)
                  : __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4d*>(
                                                   reinterpret_cast<const char*>(at) + (wm + 32 * i) * 128 + kfrag[kk]));
#pragma unroll
    for (int j = 0; j < FN; ++j)
      f.b[j] = BT ? read_tr(bt, bmn[j] + kk * 16 * 32 * 16, 32)
                  : __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4d*>(
                                                   reinterpret_cast<const char*>(bt) + (wn + 32 * j) * 128 + kfrag[kk]));
  };
  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};
  auto mma = [&](const Frags& f) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
  };

  // column sums (CS): this block's columns cs_c0 .. cs_c0 + cs_w - 1 of the
  // n-tile, thread t adds columns cs_c0 + 4 (t % ng) .. +3 of k rows t / ng,
  // t / ng + 512 / ng, .. of each stage
  const int cs_w = 4 << g.cs_shift, cs_c0 = (m0 / BM) * cs_w, ng = cs_w >> 2;
  const bool cs_blk = CS && g.colsum != nullptr && cs_c0 < 256;  // block-uniform
  const int cs_c = cs_c0 + 4 * (tid % ng), cs_k0 = tid / ng;
  float csum[4] = {0.f, 0.f, 0.f, 0.f};
  auto colsum_stage = [&](const u32x4d* st) {
    const char* bt = reinterpret_cast<const char*>(st + UNITS_A);
    for (int kr = cs_k0; kr < BKX; kr += 512 / ng) {
      const u32x2d v =
          *reinterpret_cast<const u32x2d*>(bt + (kr * 32 + ((cs_c >> 3) ^ (4 * (kr & 3)))) * 16 + (cs_c & 7) * 2);
      csum[0] += __builtin_bit_cast(float, v[0] << 16);
      csum[1] += __builtin_bit_cast(float, v[0] & 0xffff0000u);
      csum[2] += __builtin_bit_cast(float, v[1] << 16);
      csum[3] += __builtin_bit_cast(float, v[1] & 0xffff0000u);
    }
  };

  const int nst = g.K / BKX;  // even (K % 128 == 0)
  issue(S0, 0);
  d2l_sync();
  Frags fa, fb;
  read(S0, 0, fa);
  // stage s sits in buffer s % 2; fa holds its first k step on entry.  The
  // copies of stage s+1 go into the other buffer, whose stage s-1 every wave
  // finished reading before the last barrier; the fragment reads of step
  // kk+1 are issued ahead of the MFMAs of step kk.
  auto body = [&](auto BUF, int s) {
    constexpr int B = decltype(BUF)::value;
    u32x4d* cur = B == 0 ? S0 : S1;
    u32x4d* nxt = B == 0 ? S1 : S0;
    if (s + 1 < nst) issue(nxt, (s + 1) * BKX);
    read(cur, 1, fb);
    mma(fa);
    if constexpr (CS) {
      if (cs_blk) colsum_stage(cur);
    }
    read(cur, 2, fa);
    mma(fb);
    read(cur, 3, fb);
    mma(fa);
    if (s + 1 < nst) {
      // the thread's copies of stage s+1 have landed and its reads of stage s
      // are done; after the barrier every wave's are
      d2l_sync();
      read(nxt, 0, fa);
    }
    mma(fb);
  };
  using C0 = std::integral_constant<int, 0>;
  using C1 = std::integral_constant<int, 1>;
  for (int s = 0; s < nst; s += 2) {
    body(C0{}, s);
    body(C1{}, s + 1);
  }
  __syncthreads();  // every wave is done reading the stages

  if constexpr (CS) {
    if (cs_blk) {  // per owned column: the k-row group sums, added in group order
      float* red = reinterpret_cast<float*>(S0);  // [512 / ng][cs_w]
#pragma unroll
      for (int e = 0; e < 4; ++e) red[cs_k0 * cs_w + cs_c - cs_c0 + e] = csum[e];
      __syncthreads();
      const int n = n0 + cs_c0 + tid;
      if (tid < cs_w && n < g.N) {
        float t = 0.f;
        for (int j = 0; j < 512 / ng; ++j) t += red[j * cs_w + tid];
        g.colsum[n] = f32_to_bf16(t);
      }
      __syncthreads();
    }
  }

  // epilogue: fp32 (+ bias), one rounding, through LDS in halves of 64 of the
  // wave's BM/2 rows (pitch 72 elements), out as 16-byte runs; waves 0-3 stage
  // in S0, waves 4-7 in S1
  constexpr int EP = 72, CPR = 8, RPI = 8;
  static_assert(4 * 64 * EP * 2 <= Cfg::STAGE * 16, "epilogue regions exceed a stage");
  uint16_t* eb = reinterpret_cast<uint16_t*>(wave < 4 ? S0 : S1) + (wave & 3) * 64 * EP;
  const __amdgpu_buffer_rsrc_t cr = rsrc(g.c, g.c_bytes);
  float bv[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) bv[j] = BIAS ? bf16_to_f32(g.bias[n0 + wn + j * 32 + row_l]) : 0.f;
#pragma unroll
  for (int h = 0; h < FM / 2; ++h) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          eb[(ii * 32 + (v >> 2) * 8 + half_l * 4 + (v & 3)) * EP + j * 32 + row_l] =
              __builtin_bit_cast(uint16_t, (__bf16)(acc[2 * h + ii][j][v] + bv[j]));
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    const int ch = lane % CPR, col = n0 + wn + ch * 8;
#pragma unroll
    for (int it = 0; it < 64 / RPI; ++it) {
      const int rw = it * RPI + lane / CPR, row = m0 + wm + h * 64 + rw;
      const u32x4d v = *reinterpret_cast<const u32x4d*>(eb + rw * EP + ch * 8);
      __builtin_amdgcn_raw_buffer_store_b128(v, cr, (row * g.ldc + col) * 2, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
  }
}

template <bool AT, bool BT, bool BIAS>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_bf16_d2l_kernel(DenseArgs g) {
  __shared__ __attribute__((aligned(16))) u32x4d S0[D2lCfg<256>::STAGE];
  __shared__ __attribute__((aligned(16))) u32x4d S1[D2lCfg<256>::STAGE];
  d2l_tile<256, AT, BT, BIAS, false>(g, xcd_block(g.tiles_m * g.tiles_n), S0, S1);
}

// Two products in one launch on 128 x 256 tiles (Linear's dX, K-major x
// K-major, and dW, MN-major x MN-major with the bias gradient's column sums):
// blocks 0 .. T0-1 take the first product's tiles, the rest the second's.
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_bf16_d2l_pair_kernel(DenseArgs g0, DenseArgs g1) {
  __shared__ __attribute__((aligned(16))) u32x4d S0[D2lCfg<128>::STAGE];
  __shared__ __attribute__((aligned(16))) u32x4d S1[D2lCfg<128>::STAGE];
  const int t0 = g0.tiles_m * g0.tiles_n, h = blockIdx.x;
  if (h < t0)
    d2l_tile<128, false, false, false, false>(g0, xcd_map(h, t0), S0, S1);
  else
    d2l_tile<128, true, true, false, true>(g1, xcd_map(h - t0, g1.tiles_m * g1.tiles_n), S0, S1);
}

bool fits(long bytes) { return bytes >= 0 && bytes < (1L << 31) - 64; }

template <int BM, int BN, bool BIAS, bool PC, bool AT, bool BT>
int launch_gemm(const DenseArgs& a0, hipStream_t st) {
  using Cfg = DenseCfg<BM, BN, AT, BT>;
  auto kern = gemm_bf16_kernel<BM, BN, BIAS, PC, AT, BT>;
  const size_t lds = Cfg::lds_bytes(PC);
  VH_LDS_LIMIT_ONCE(kern);
  DenseArgs a = a0;
  a.tiles_m = (a.M + BM - 1) / BM;
  a.tiles_n = (a.N + BN - 1) / BN;
  a.cs_shift = colsum_shift(a.tiles_m, BN);
  kern<<<dim3((unsigned)(a.tiles_m * a.tiles_n)), PC ? 512 : 256, lds, st>>>(a);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

// 128 x 256 tiles (one block per CU, producer / consumer form, 64 x 128 per
// consumer wave) when the grid still fills the chip, else 128 x 128 (two
// blocks per CU of four waves that both load and multiply: already two waves
// per SIMD, and measured as fast as or faster than a split form)
template <bool AT, bool BT>
int launch_layout(const DenseArgs& g, bool big, hipStream_t st) {
  if (big)
    return g.bias ? launch_gemm<128, 256, true, true, AT, BT>(g, st) : launch_gemm<128, 256, false, true, AT, BT>(g, st);
  return g.bias ? launch_gemm<128, 128, true, false, AT, BT>(g, st) : launch_gemm<128, 128, false, false, AT, BT>(g, st);
}

}  // namespace

bool dense_bf16_ok(long M, long N, long K, bool at, long lda, bool bt, long ldb, long ldc, const void* a,
                   const void* b, const void* c) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 8 || lda % 8 || ldb % 8) return false;
  if ((at && (M % 8 || lda < M)) || (bt && (N % 8 || ldb < N)) || (!at && lda < K) || (!bt && ldb < K)) return false;
  if (((uintptr_t)a & 15) || ((uintptr_t)b & 15) || ((uintptr_t)c & 1)) return false;
  return fits((at ? K : M) * lda * 2) && fits((bt ? K : N) * ldb * 2) && fits(M * ldc * 2);
}

namespace {
DenseArgs dense_args(const void* a, int lda, bool at, const void* b, int ldb, bool bt, void* c, int ldc, int M,
                     int N, int K, const void* bias, void* colsum) {
  DenseArgs g{};
  g.colsum = (uint16_t*)colsum;
  g.vec_epi = ((uintptr_t)c & 15) == 0 && ldc % 8 == 0 && N % 8 == 0;
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
  g.a_bytes = (int)((long)(at ? K : M) * lda * 2);
  g.b_bytes = (int)((long)(bt ? K : N) * ldb * 2);
  g.c_bytes = (int)((long)M * ldc * 2);
  return g;
}

// 128 x 256 tiles when they still give at least one block per CU
bool dense_big(int M, int N) { return (long)((M + 127) / 128) * ((N + 255) / 256) >= 256; }

// The 256 x 256 direct-to-LDS kernel: whole tiles only (no bounds checks in
// its loads or stores), K in whole stages, 16-byte aligned rows of every
// operand, and a grid of at least one block per CU.
bool dense_d2l(const DenseArgs& g, bool colsum) {
  return !colsum && g.M % 256 == 0 && g.N % 256 == 0 && g.K % (2 * kD2lBK) == 0 && g.vec_epi &&
         (long)(g.M / 256) * (g.N / 256) >= 256;
}

template <bool AT, bool BT>
int launch_d2l(const DenseArgs& a0, hipStream_t st) {
  DenseArgs a = a0;
  a.tiles_m = a.M / 256;
  a.tiles_n = a.N / 256;
  auto kern = a.bias ? gemm_bf16_d2l_kernel<AT, BT, true> : gemm_bf16_d2l_kernel<AT, BT, false>;
  kern<<<dim3((unsigned)(a.tiles_m * a.tiles_n)), 512, 0, st>>>(a);
  VH_LAUNCH_CHECK();
  return VH_OK;
}
}  // namespace

int dense_bf16_gemm(const void* a, int lda, bool at, const void* b, int ldb, bool bt, void* c, int ldc, int M,
                    int N, int K, const void* bias, hipStream_t st, void* colsum) {
  const bool big = dense_big(M, N);
  if (colsum && (!bt || bias)) return VH_ERR_UNSUPPORTED;
  const DenseArgs g = dense_args(a, lda, at, b, ldb, bt, c, ldc, M, N, K, bias, colsum);
  if (dense_d2l(g, colsum != nullptr)) {
    if (at) return bt ? launch_d2l<true, true>(g, st) : launch_d2l<true, false>(g, st);
    return bt ? launch_d2l<false, true>(g, st) : launch_d2l<false, false>(g, st);
  }
  if (at) return bt ? launch_layout<true, true>(g, big, st) : launch_layout<true, false>(g, big, st);
  return bt ? launch_layout<false, true>(g, big, st) : launch_layout<false, false>(g, big, st);
}

namespace {
int launch_d2l_pair(DenseArgs a0, DenseArgs a1, hipStream_t st) {
  for (DenseArgs* a : {&a0, &a1}) {
    a->tiles_m = a->M / 128;
    a->tiles_n = a->N / 256;
    a->cs_shift = colsum_shift(a->tiles_m, 256);
  }
  gemm_bf16_d2l_pair_kernel<<<dim3((unsigned)(a0.tiles_m * a0.tiles_n + a1.tiles_m * a1.tiles_n)), 512, 0, st>>>(a0,
                                                                                                                 a1);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <int BN, bool PC>
int launch_pair(DenseArgs a0, DenseArgs a1, hipStream_t st) {
  for (DenseArgs* a : {&a0, &a1}) {
    a->tiles_m = (a->M + 127) / 128;
    a->tiles_n = (a->N + BN - 1) / BN;
    a->cs_shift = colsum_shift(a->tiles_m, BN);
  }
  auto kern = gemm_bf16_pair_kernel<BN, PC, false, false, true, true>;
  const size_t lds = std::max(DenseCfg<128, BN, false, false>::lds_bytes(PC), DenseCfg<128, BN, true, true>::lds_bytes(PC));
  VH_LDS_LIMIT_ONCE(kern);
  kern<<<dim3((unsigned)(a0.tiles_m * a0.tiles_n + a1.tiles_m * a1.tiles_n)), PC ? 512 : 256, lds, st>>>(a0, a1);
  VH_LAUNCH_CHECK();
  return VH_OK;
}
}  // namespace

int dense_bf16_gemm_pair(const DenseProblem& p0, const DenseProblem& p1, hipStream_t st) {
  // the pair form serves a K-major x K-major product next to an MN-major x
  // MN-major one (Linear's dX and dW)
  if (p0.at || p0.bt || !p1.at || !p1.bt || p0.colsum) return VH_ERR_UNSUPPORTED;
  const DenseArgs a0 = dense_args(p0.a, p0.lda, p0.at, p0.b, p0.ldb, p0.bt, p0.c, p0.ldc, p0.M, p0.N, p0.K, nullptr,
                                  nullptr);
  const DenseArgs a1 = dense_args(p1.a, p1.lda, p1.at, p1.b, p1.ldb, p1.bt, p1.c, p1.ldc, p1.M, p1.N, p1.K, nullptr,
                                  p1.colsum);
  // whole 128 x 256 tiles of both, at least one block per CU: the
  // direct-to-LDS pair kernel
  auto whole = [](const DenseArgs& g) {
    return g.M % 128 == 0 && g.N % 256 == 0 && g.K % (2 * kD2lBK) == 0 && g.vec_epi != 0;
  };
  if (whole(a0) && whole(a1) && (long)(a0.M / 128) * (a0.N / 256) + (long)(a1.M / 128) * (a1.N / 256) >= 256)
    return launch_d2l_pair(a0, a1, st);
  const long t256 = (long)((p0.M + 127) / 128) * ((p0.N + 255) / 256) + (long)((p1.M + 127) / 128) * ((p1.N + 255) / 256);
  return t256 >= 256 ? launch_pair<256, true>(a0, a1, st) : launch_pair<128, false>(a0, a1, st);
}

}  // namespace vh
