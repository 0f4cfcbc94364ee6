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
  float* colsum;      // [N] or nullptr: column sums of an MN-major B over K (pair kernel)
  int M, N, K, lda, ldb, ldc;
  int a_bytes, b_bytes, c_bytes;
  int tiles_m, tiles_n;
  int cs_shift;       // column-sum ownership: 4 << cs_shift columns per block
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

// ---------------------------------------------------------------- BM x 256 tiles, direct-to-LDS loads
// For products whose tiles are whole (M a multiple of BM, N of 256, K of 64):
// a product on 256 x 256 tiles, or a Linear layer's dX and dW as one launch on
// 128 x 256 tiles.  The operands are copied from global memory straight into
// LDS (buffer_load_dwordx4 ... lds: no registers, no LDS store instructions),
// two LDS stages of 32 k, the copies of stage s+1 issued when stage s starts;
// eight waves split the tile 2 (m) x 4 (n), BM/2 x 64 per wave (fragments of
// 32 x 32, two waves per SIMD).  A stage holds BM + 256 rows of 128 bytes,
// laid out as for the bf16 kernels (the lane -> global unit map sets the
// layout: LDS DMA lands lane l at unit l of the instruction's base):
//  * K-major tile (rows of 8 units of 4 k): slot t of row r holds k unit
//    t ^ ((r >> 1) & 7); a fragment read is one ds_read_b128 per lane, 16
//    consecutive lanes on 16 distinct 16-byte bank groups.
//  * MN-major tile (32 k rows of R/4 units): slot t of k row kr holds row unit
//    t ^ (8 (kr & 1)); a fragment read is one ds_read_b32 per lane, the two k
//    rows of an MFMA step on the two bank halves.
// Within a 4-k unit the MFMA's two k lanes take k 2t + (lane / 32) in step t,
// so one 16-byte K-major read serves both steps of the unit.
constexpr int kF32D2lBK = 32;  // k per stage

// s_waitcnt vmcnt(0) lgkmcnt(0), then the block barrier
__device__ __forceinline__ void f32_d2l_sync() {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int BM>
struct F32D2lCfg {
  static constexpr int FM = BM / 64, FN = 2;              // 32 x 32 fragments per wave
  static constexpr int A_UNITS = BM * 8, B_UNITS = 2048;   // 16-byte units per stage
  static constexpr int STAGE = A_UNITS + B_UNITS;
  static constexpr int ACPW = BM / 64, BCPW = 4;           // copy instructions per wave and stage
};

// One BM x 256 tile of C = A . B (logical block lb), S0 / S1 the two stages.
// CS: the column sums of an MN-major B over K (a Linear weight gradient's bias
// gradient) from the staged tiles: the tiles_m blocks of a column tile each
// own 4 << cs_shift of its columns, so every column is summed by exactly one
// block over all K; a thread adds 4 consecutive owned columns of one k row per
// stage, in stage order, and the k-row group sums are added in group order.
template <int BM, bool AT, bool BT, bool BIAS, bool CS>
__device__ __forceinline__ void f32_d2l_tile(const DenseF32Args& g, const int lb, u32x4f* S0, u32x4f* S1) {
  using Cfg = F32D2lCfg<BM>;
  constexpr int FM = Cfg::FM, FN = Cfg::FN, UNITS_A = Cfg::A_UNITS;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave >> 2) * (BM / 2), wn = (wave & 3) * 64;
  const int grp = lb / (kGroupMf * g.tiles_n), first_m = grp * kGroupMf;
  const int gm = min(g.tiles_m - first_m, kGroupMf);
  const int in_grp = lb - grp * kGroupMf * g.tiles_n;
  const int m0 = (first_m + in_grp % gm) * BM, n0 = (in_grp / gm) * 256;

  // copy instruction c of an operand with R rows (R = BM or 256):
  //  K-major: rows 8c .. 8c+7, lane -> row 8c + lane/8, slot lane%8 holds k
  //    unit (lane%8) ^ ((row >> 1) & 7);
  //  MN-major (UR = R/4 units per k row): k rows (64/UR) c .., lane -> k row
  //    (64/UR) c + lane/UR, slot lane%UR holds row unit slot ^ (8 (kr & 1)).
  auto unit_off = [&](bool mn, int R, int rc0, int ld, int c) {
    if (!mn) {
      const int r = 8 * c + (lane >> 3), u = (lane & 7) ^ ((r >> 1) & 7);
      return ((rc0 + r) * ld + 4 * u) * 4;
    }
    const int UR = R / 4;
    const int kr = (64 / UR) * c + lane / UR, mu = (lane % UR) ^ (8 * (kr & 1));
    return (kr * ld + rc0 + 4 * mu) * 4;
  };
  int aoff[Cfg::ACPW], boff[Cfg::BCPW];
#pragma unroll
  for (int i = 0; i < Cfg::ACPW; ++i) aoff[i] = unit_off(AT, BM, m0, g.lda, Cfg::ACPW * wave + i);
#pragma unroll
  for (int i = 0; i < Cfg::BCPW; ++i) boff[i] = unit_off(BT, 256, n0, g.ldb, Cfg::BCPW * wave + i);
  const __amdgpu_buffer_rsrc_t ar = rsrc_f(g.a, g.a_bytes), br = rsrc_f(g.b, g.b_bytes);
  auto issue = [&](u32x4f* st, int k0) {
    const int ask = __builtin_amdgcn_readfirstlane(AT ? k0 * g.lda * 4 : k0 * 4);
    const int bsk = __builtin_amdgcn_readfirstlane(BT ? k0 * g.ldb * 4 : k0 * 4);
    const uint32_t la = lds_byte_addr(st);
#pragma unroll
    for (int i = 0; i < Cfg::ACPW; ++i) lds_copy16(ar, aoff[i], ask, la + (Cfg::ACPW * wave + i) * 64 * 16);
#pragma unroll
    for (int i = 0; i < Cfg::BCPW; ++i) lds_copy16(br, boff[i], bsk, la + (UNITS_A + (Cfg::BCPW * wave + i) * 64) * 16);
  };

  // fragment reads of k unit q (0 .. 7) of a stage: per fragment the values of
  // steps t = 0, 1 (k 4q + 2t + half_l)
  const int row_l = lane & 31, half_l = lane >> 5;
  const int kb = (8 * row_l + ((row_l >> 1) & 7)) * 16;  // K-major: row row_l, slot 0 ^ swizzle
  const int kx = ((row_l >> 1) & 7);
  struct Frags {
    float a[FM][2], b[FN][2];
  };
  auto mn_val = [&](const char* t, int UR, int r, int kr) {
    return *reinterpret_cast<const float*>(t + (kr * UR + ((r >> 2) ^ (8 * (kr & 1)))) * 16 + (r & 3) * 4);
  };
  auto read = [&](const u32x4f* st, int q, Frags& f) {
    const char* at = reinterpret_cast<const char*>(st);
    const char* bt = reinterpret_cast<const char*>(st + UNITS_A);
    const int kq = kb + ((q ^ kx) - kx) * 16;  // slot q ^ ((row_l >> 1) & 7)
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      if constexpr (AT) {
#pragma unroll
        for (int t = 0; t < 2; ++t) f.a[i][t] = mn_val(at, BM / 4, wm + 32 * i + row_l, 4 * q + 2 * t + half_l);
      } else {
        const u32x4f v = *reinterpret_cast<const u32x4f*>(at + (wm + 32 * i) * 128 + kq);
        f.a[i][0] = __builtin_bit_cast(float, half_l ? v[1] : v[0]);
        f.a[i][1] = __builtin_bit_cast(float, half_l ? v[3] : v[2]);
      }
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      if constexpr (BT) {
#pragma unroll
        for (int t = 0; t < 2; ++t) f.b[j][t] = mn_val(bt, 64, wn + 32 * j + row_l, 4 * q + 2 * t + half_l);
      } else {
        const u32x4f v = *reinterpret_cast<const u32x4f*>(bt + (wn + 32 * j) * 128 + kq);
        f.b[j][0] = __builtin_bit_cast(float, half_l ? v[1] : v[0]);
        f.b[j][1] = __builtin_bit_cast(float, half_l ? v[3] : v[2]);
      }
    }
  };
  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};
  auto mma = [&](const Frags& f) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[i][t], f.b[j][t], acc[i][j], 0, 0, 0);
  };

  // column sums (CS): this block's columns cs_c0 .. cs_c0 + cs_w - 1 of the
  // n-tile; thread t adds columns cs_c0 + 4 (t % ng) .. +3 of k rows t / ng,
  // t / ng + 512 / ng, .. of each stage
  const int cs_w = 4 << g.cs_shift, cs_c0 = (m0 / BM) * cs_w, ng = cs_w >> 2;
  const bool cs_blk = CS && g.colsum != nullptr && cs_c0 < 256;  // block-uniform
  const int cs_c = cs_c0 + 4 * (tid % ng), cs_k0 = tid / ng;
  float csum[4] = {0.f, 0.f, 0.f, 0.f};
  auto colsum_stage = [&](const u32x4f* st) {
    const char* bt = reinterpret_cast<const char*>(st + UNITS_A);
    for (int kr = cs_k0; kr < kF32D2lBK; kr += 512 / ng) {
      const u32x4f v = *reinterpret_cast<const u32x4f*>(bt + (kr * 64 + ((cs_c >> 2) ^ (8 * (kr & 1)))) * 16);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t u = v[e];  // (a vector element is not an object: bit-cast a copy)
        csum[e] += __builtin_bit_cast(float, u);
      }
    }
  };

  const int nst = g.K / kF32D2lBK;  // even (K % 64 == 0)
  issue(S0, 0);
  f32_d2l_sync();
  Frags fa, fb;
  read(S0, 0, fa);
  // stage s sits in buffer s % 2; fa holds its first unit on entry.  The copies
  // of stage s+1 go into the other buffer, whose stage s-1 every wave finished
  // reading before the last barrier; the reads of unit q+1 are issued ahead of
  // the MFMAs of unit q.
  auto body = [&](auto BUF, int s) {
    constexpr int B = decltype(BUF)::value;
    u32x4f* cur = B == 0 ? S0 : S1;
    u32x4f* nxt = B == 0 ? S1 : S0;
    if (s + 1 < nst) issue(nxt, (s + 1) * kF32D2lBK);
    read(cur, 1, fb);
    mma(fa);
    if constexpr (CS) {
      if (cs_blk) colsum_stage(cur);
    }
#pragma unroll
    for (int q = 2; q < 8; q += 2) {
      read(cur, q, fa);
      mma(fb);
      read(cur, q + 1, fb);
      mma(fa);
    }
    if (s + 1 < nst) {
      f32_d2l_sync();
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

  if constexpr (CS) {
    if (cs_blk) {  // per owned column: the k-row group sums, added in group order
      __syncthreads();  // every wave is done reading the stages
      float* red = reinterpret_cast<float*>(S0);  // [512 / ng][cs_w]
#pragma unroll
      for (int e = 0; e < 4; ++e) red[cs_k0 * cs_w + cs_c - cs_c0 + e] = csum[e];
      __syncthreads();
      const int n = n0 + cs_c0 + tid;
      if (tid < cs_w && n < g.N) {
        float t = 0.f;
        for (int j = 0; j < 512 / ng; ++j) t += red[j * cs_w + tid];
        g.colsum[n] = t;
      }
    }
  }

  // epilogue: (+ bias) fp32 stores, lanes walk columns (32 columns x 2 rows per store)
  const __amdgpu_buffer_rsrc_t cr = rsrc_f(g.c, g.c_bytes);
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int col = n0 + wn + j * 32 + row_l;
    const float bv = BIAS ? g.bias[col] : 0.f;
    const int voff = (col + half_l * 4 * g.ldc) * 4;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm + i * 32 + (v >> 2) * 8 + (v & 3);  // + 4 * half_l
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, acc[i][j][v] + bv), cr, voff,
                                              row * g.ldc * 4, 0);
      }
  }
}

template <bool AT, bool BT, bool BIAS>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_f32_d2l_kernel(DenseF32Args g) {
  __shared__ __attribute__((aligned(16))) u32x4f S0[F32D2lCfg<256>::STAGE];
  __shared__ __attribute__((aligned(16))) u32x4f S1[F32D2lCfg<256>::STAGE];
  f32_d2l_tile<256, AT, BT, BIAS, false>(g, xcd_block(g.tiles_m * g.tiles_n), S0, S1);
}

// Two products in one launch on 128 x 256 tiles (Linear's dX, K-major x
// K-major, and dW, MN-major x MN-major with the bias gradient's column sums):
// blocks 0 .. T0-1 take the first product's tiles, the rest the second's.
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_f32_d2l_pair_kernel(DenseF32Args g0, DenseF32Args g1) {
  __shared__ __attribute__((aligned(16))) u32x4f S0[F32D2lCfg<128>::STAGE];
  __shared__ __attribute__((aligned(16))) u32x4f S1[F32D2lCfg<128>::STAGE];
  const int t0 = g0.tiles_m * g0.tiles_n, h = blockIdx.x;
  if (h < t0)
    f32_d2l_tile<128, false, false, false, false>(g0, xcd_map(h, t0), S0, S1);
  else
    f32_d2l_tile<128, true, true, false, true>(g1, xcd_map(h - t0, g1.tiles_m * g1.tiles_n), S0, S1);
}

template <bool AT, bool BT>
int launch_f32_d2l(const DenseF32Args& a0, hipStream_t st) {
  DenseF32Args a = a0;
  a.tiles_m = a.M / 256;
  a.tiles_n = a.N / 256;
  const dim3 grid((unsigned)(a.tiles_m * a.tiles_n));
  if (a.bias)
    gemm_f32_d2l_kernel<AT, BT, true><<<grid, 512, 0, st>>>(a);
  else
    gemm_f32_d2l_kernel<AT, BT, false><<<grid, 512, 0, st>>>(a);
  VH_LAUNCH_CHECK();
  return VH_OK;
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

namespace {
DenseF32Args f32_args(const void* a, int lda, bool at, const void* b, int ldb, bool bt, void* c, int ldc, int M,
                      int N, int K, const void* bias) {
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
  return g;
}
}  // namespace

int dense_f32_gemm_pair(const DenseProblem& p0, const DenseProblem& p1, hipStream_t st) {
  // Linear's dX (K-major x K-major) next to its dW (MN-major x MN-major, with
  // the bias gradient as column sums of dY): whole 128 x 256 tiles of both,
  // at least one block per CU, 16-byte aligned operand rows
  if (p0.at || p0.bt || !p1.at || !p1.bt || p0.colsum) return VH_ERR_UNSUPPORTED;
  for (const DenseProblem* p : {&p0, &p1})
    if (p->M % 128 || p->N % 256 || p->K % (2 * kF32D2lBK) || p->lda % 4 || p->ldb % 4) return VH_ERR_UNSUPPORTED;
  if ((long)(p0.M / 128) * (p0.N / 256) + (long)(p1.M / 128) * (p1.N / 256) < 256) return VH_ERR_UNSUPPORTED;
  DenseF32Args a0 = f32_args(p0.a, p0.lda, false, p0.b, p0.ldb, false, p0.c, p0.ldc, p0.M, p0.N, p0.K, nullptr);
  DenseF32Args a1 = f32_args(p1.a, p1.lda, true, p1.b, p1.ldb, true, p1.c, p1.ldc, p1.M, p1.N, p1.K, nullptr);
  a1.colsum = (float*)p1.colsum;
  for (DenseF32Args* a : {&a0, &a1}) {
    a->tiles_m = a->M / 128;
    a->tiles_n = a->N / 256;
    a->cs_shift = colsum_shift(a->tiles_m, 256);
  }
  gemm_f32_d2l_pair_kernel<<<dim3((unsigned)(a0.tiles_m * a0.tiles_n + a1.tiles_m * a1.tiles_n)), 512, 0, st>>>(a0,
                                                                                                                a1);
  VH_LAUNCH_CHECK();
  return VH_OK;
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
  // whole 256 x 256 tiles that fill the chip: the direct-to-LDS kernel
  // (16-byte aligned operand rows; the stores are 4-byte)
  if (M % 256 == 0 && N % 256 == 0 && K % (2 * kF32D2lBK) == 0 && lda % 4 == 0 && ldb % 4 == 0 &&
      (long)(M / 256) * (N / 256) >= 256) {
    if (at) return bt ? launch_f32_d2l<true, true>(g, st) : launch_f32_d2l<true, false>(g, st);
    return bt ? launch_f32_d2l<false, true>(g, st) : launch_f32_d2l<false, false>(g, st);
  }
  const bool big = (long)((M + 127) / 128) * ((N + 127) / 128) >= 512;
  if (at) return bt ? launch_layout_f32<true, true>(g, big, st) : launch_layout_f32<true, false>(g, big, st);
  return bt ? launch_layout_f32<false, true>(g, big, st) : launch_layout_f32<false, false>(g, big, st);
}

}  // namespace vh
