// vh_wgrad.hip -- bf16 weight gradient of stride-1 3x3 convolutions on NCHW
// tensors, gfx950 MFMA (v_mfma_f32_32x32x16_bf16).
//
//   dW[o][c][r][s] = sum_{n,p,q} dY[n][o][p][q] * x[n][c][p+r-ph][q+s-pw]
//
// GEMM view: rows = o, columns = (c, tap), K = positions.  Both operands are
// K-contiguous in NCHW memory (positions run along rows), so rows of dY and x
// are copied to LDS as they are -- no transposition, aligned vector stores.
// The K walk runs over the x columns v of G output rows: with q = v + pw - s,
//   dW[o][c][r][s] = sum_{g,v} dY[o][g][v + pw - s] * x[c][g + r][v],
// so one aligned 16-byte read of an x row serves all three s taps of a row r,
// and the three dY windows (shifts pw - s = +1, 0, -1 for pw = 1) are built
// from three aligned 16-byte reads of the dY row and a byte-align funnel shift.
// dY rows sit in LDS with at least 8 zero elements between them (and before the
// first), so windows that run past a row end read zeros.
//
// A block stages, per K step,
//   * dY rows [64 o][8 + G*DP]   (row g of o at 8 + g*DP, zero gaps), and
//   * x rows  [64 c][(G+2)*XP]   (input rows p0-ph .. p0+G+1-ph, zero past W),
// in two LDS buffers (loads for step k+1 are in flight while step k runs).
// Each wave accumulates a 32(o) x 32(c) x 9-tap tile in AGPRs.  Split-K: the
// grid's z dimension walks disjoint ranges of K steps; partial sums go to an
// fp32 workspace in the accumulators' own layout
//   [split][tile][wave][tap][row group j][lane][4]   (element v = 4j + k of lane)
// written as one 16-byte store per lane and (tap, j), and a second kernel adds
// them in a fixed order and writes dW (OIHW).  The optional bias gradient (sum of dY over
// positions) is accumulated by the c-tile-0 blocks from the same LDS copy of dY.
#include <algorithm>
#include <type_traits>

#include "vh_kernels.hpp"

namespace vh {

#define VH_TRY_W(expr)          \
  do {                          \
    int _s = (expr);            \
    if (_s != VH_OK) return _s; \
  } while (0)

typedef unsigned int u32x4w __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2w __attribute__((ext_vector_type(2)));

struct WgradArgs {
  const uint16_t* dy;  // [N][O][P][Q]
  const uint16_t* x;   // [N][C][H][W]
  float* part;         // [splits][RS][O][C]
  float* dbias_part;   // [splits][O] or nullptr
  int N, C, H, W, O, P, Q, ph, pw;
  int G;               // output rows per K step (divides P)
  int XV;              // x columns walked per row and step (segment width): multiple of 8
  int nseg;            // column segments per row (1: whole rows)
  int HL;              // dY columns loaded left of the segment: 0 (whole rows) or 8
  int BW;              // dY columns per row slot summed for the bias gradient (multiple of 8)
  int RL, XL;          // dY / x elements loaded per row and step
  int DP;              // LDS pitch of a dY row (elements)
  int XP;              // LDS pitch of an x row (elements): XV
  int OS, CS;          // LDS strides per o / per c (elements)
  int steps_per_img;   // P / G
  int total_steps;     // N * steps_per_img
  int steps_per_split;
  int V;               // elements per global load (8, 4 or 2): divides Q and W
  int cpr_dy, cpr_x;   // chunks of V elements per dY row / per x row
  int dadv, cadv;      // TPO*V elements (an item's stride) of a dY owner's run as (rows, columns), < RL
  int xadv, xcadv;     // the same for x rows (columns < XL)
  int dy_bytes, x_bytes;  // buffer ranges (< 2^31)
  int tiles_o, tiles_c, splits;       // grid = tiles_o * tiles_c * splits blocks
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

template <int V>
struct VecT;
template <> struct VecT<8> { using t = u32x4w; };
template <> struct VecT<4> { using t = u32x2w; };
template <> struct VecT<2> { using t = uint32_t; };

__device__ __forceinline__ uint32_t funnel16(uint32_t lo, uint32_t hi) {
  // bytes 2..5 of (hi:lo): upper bf16 of lo, lower bf16 of hi
  return __builtin_amdgcn_alignbyte(hi, lo, 2);
}

// 8 consecutive bf16 starting SH elements into the 24-element window (c0, c1, c2)
template <int SH>
__device__ __forceinline__ u32x4w window8(const u32x4w& c0, const u32x4w& c1, const u32x4w& c2) {
  if constexpr (SH >= 8) {
    return window8<SH - 8>(c1, c2, c2);
  } else if constexpr (SH == 0) {
    return c0;
  } else if constexpr (SH == 2) {
    return u32x4w{c0.y, c0.z, c0.w, c1.x};
  } else if constexpr (SH == 4) {
    return u32x4w{c0.z, c0.w, c1.x, c1.y};
  } else if constexpr (SH == 6) {
    return u32x4w{c0.w, c1.x, c1.y, c1.z};
  } else if constexpr (SH == 1) {
    return u32x4w{funnel16(c0.x, c0.y), funnel16(c0.y, c0.z), funnel16(c0.z, c0.w), funnel16(c0.w, c1.x)};
  } else if constexpr (SH == 3) {
    return u32x4w{funnel16(c0.y, c0.z), funnel16(c0.z, c0.w), funnel16(c0.w, c1.x), funnel16(c1.x, c1.y)};
  } else if constexpr (SH == 5) {
    return u32x4w{funnel16(c0.z, c0.w), funnel16(c0.w, c1.x), funnel16(c1.x, c1.y), funnel16(c1.y, c1.z)};
  } else {  // 7
    return u32x4w{funnel16(c0.w, c1.x), funnel16(c1.x, c1.y), funnel16(c1.y, c1.z), funnel16(c1.z, c1.w)};
  }
}

// Load items: thread t serves row owner t/4 (an o of the dY tile, a c of the x
// tile) and takes that owner's chunks t%4, t%4 + 4, ...; chunk k of a dY owner
// is row k / cpr, column (k % cpr) * V.  Offsets advance incrementally.
// PC: 512 threads, waves 0-3 multiply (consumers), waves 4-7 only
// load and store into LDS (producers, threads 256-511 serving the item map of
// threads 0-255).  Neither role holds the other's registers, so two waves fit
// per SIMD and the loads run beside the MFMAs of the other role.
// KQ (K quarters; whole rows, producer / consumer form): the block tile is
// 32 o x 32 c, and the four consumer waves share it, each taking every fourth
// 16-position MFMA step of each K step; at the end the four accumulator sets
// are summed in LDS in wave order and one partial tile is stored.  Against the
// 64 x 64 tile that is a quarter of the split-K partial bytes for the same
// number of blocks, for twice the operand rows staged per MFMA.
template <int R, int S, int PW, int V, int ND, int NX, bool SEG, int DEPTH, bool PC = false, bool KQ = false>
__global__ __launch_bounds__(PC ? 512 : 256) void wgrad_rows_bf16_kernel(WgradArgs a) {
  static_assert(R == 3 && S == 3, "3x3 windows");
  static_assert(!KQ || (PC && !SEG), "K quarters: whole rows, producer / consumer blocks");
  constexpr int RS = R * S;
  constexpr int TO = KQ ? 32 : 64, TC = KQ ? 32 : 64;  // block tile (o, c)
  constexpr int TPO = 256 / TO;                        // load threads per row owner
  using VT = typename VecT<V>::t;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  const bool producer = PC && threadIdx.x >= 256;
  const int tid = PC ? (int)(threadIdx.x & 255u) : (int)threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar) index
  const int wo = KQ ? 0 : (wave >> 1) * 32, wc = KQ ? 0 : (wave & 1) * 32;
  // logical block -> (o tile, c tile, split): the tiles of one split (which
  // read the same dY / x rows) are consecutive, hence on one XCD's L2
  const int lb = xcd_block(a.tiles_o * a.tiles_c * a.splits);
  const int tile = lb % (a.tiles_o * a.tiles_c), split = lb / (a.tiles_o * a.tiles_c);
  const int tile_c = tile / a.tiles_o;
  const int o0 = (tile % a.tiles_o) * TO, c0 = tile_c * TC;
  const int G = a.G, DP = a.DP, XP = a.XP, OS = a.OS, CS = a.CS;
  const int XR = G + R - 1;
  const int dy_elems = TO * OS, x_elems = TC * CS;
  const int stage = dy_elems + x_elems + 8;  // elements per stage (the last 8: a sink
                                             // for the stores of unused load items)
#define DYS(st) (smem + (st) * stage)
#define XS(st) (smem + (st) * stage + dy_elems)

  const int step_b = split * a.steps_per_split;
  const int step_e = min(a.total_steps, step_b + a.steps_per_split);
  const int nsteps = max(0, step_e - step_b);

  // zero both stages once: gaps and padding are never written by the loader
  for (int i = threadIdx.x; i < 2 * stage / 8; i += PC ? 512 : 256)
    reinterpret_cast<u32x4w*>(smem)[i] = u32x4w{0u, 0u, 0u, 0u};

  const int PQ = a.P * a.Q, HW = a.H * a.W;
  const int own = tid / TPO, sub = tid % TPO;
  // dY owner o = own: chunk k = sub + 4*it -> (row g, column) ; x owner c = own likewise
  const bool dy_own_ok = o0 + own < a.O, x_own_ok = c0 + own < a.C;
  const int dy_base_g = dy_own_ok ? (o0 + own) * PQ * 2 : 0;  // bytes, plane of o at image 0
  const int x_base_g = x_own_ok ? (c0 + own) * HW * 2 : 0;
  const int dy_chunks = G * a.cpr_dy, x_chunks = XR * a.cpr_x;
  // item it of this thread is chunk sub + TPO*it of its owner: (row, column) start
  // at (g0, col0) and advance by TPO*V elements per item (a.dadv rows + a.cadv
  // columns, with one carry); recomputed per step instead of kept in registers
  int dg0 = 0, dc0 = sub * V;
  while (dc0 >= a.RL) { dc0 -= a.RL; ++dg0; }
  int xj0 = 0, xc0 = sub * V;
  while (xc0 >= a.XL) { xc0 -= a.XL; ++xj0; }
  const __amdgpu_buffer_rsrc_t dyr = __builtin_amdgcn_make_buffer_rsrc((void*)a.dy, (short)0, a.dy_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t xrr = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.x_bytes, 0x00020000);

  // Whole rows: an owner's dY run (G rows) and x run (G+2 rows) are contiguous
  // in global memory, so item it sits at a fixed offset it*4V elements from the
  // thread's first item; only the LDS slot of each item and, for x, its run row
  // (whose validity moves with the step) are kept, computed once.  Unused items
  // and owners past O / C go to the sink / load zeros.
  constexpr int kSinkRow = 1 << 20;
  int d_lds[SEG ? 1 : ND], x_lds[SEG ? 1 : NX], x_row[SEG ? 1 : NX];
  const int sink_el = dy_elems + x_elems;  // the stage's sink, relative to the stage
  if constexpr (!SEG) {
    int g = dg0, col = dc0;
#pragma unroll
    for (int it = 0; it < ND; ++it) {
      d_lds[it] = sub + TPO * it < dy_chunks ? own * OS + 8 + g * DP + col : sink_el;
      col += a.cadv;
      const int wrap = col >= a.RL;
      col -= wrap ? a.RL : 0;
      g += a.dadv + wrap;
    }
    int j = xj0;
    col = xc0;
#pragma unroll
    for (int it = 0; it < NX; ++it) {
      const bool ok = sub + TPO * it < x_chunks;
      x_lds[it] = ok ? dy_elems + own * CS + j * XP + col : sink_el;
      x_row[it] = ok && x_own_ok ? j : kSinkRow;
      col += a.xcadv;
      const int wrap = col >= a.XL;
      col -= wrap ? a.XL : 0;
      j += a.xadv + wrap;
    }
  }
  const int d_voff = dy_own_ok ? dy_base_g + sub * V * 2 : (int)0x80000000u;
  const int x_voff = x_base_g + sub * V * 2;

  // DEPTH register sets: with two, the loads of step k+2 are in flight while
  // step k is multiplied and step k+1 is written to LDS
  VT rdy[DEPTH][ND], rx[DEPTH][NX];
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, DEPTH - 1>;
  // Branch-free load / store sequences (selects, and a sink slot in LDS for
  // unused items), so the compiler can count outstanding loads exactly.
  auto gload = [&](auto SET, int step) {
    constexpr int sI = decltype(SET)::value;
    if constexpr (!SEG) {
      const int n = step / a.steps_per_img;
      const int p0 = (step - n * a.steps_per_img) * G;
      const int dstep = (n * a.O * PQ + p0 * a.Q) * 2;  // scalar byte offset of the dY run
#pragma unroll
      for (int it = 0; it < ND; ++it)
        rdy[sI][it] = BufLoad<V>::ld(dyr, d_voff + it * 2 * TPO * V, dstep);
      // x run row j is input row p0 - ph + j; t = byte offset of the thread's first item
      const int rbase = p0 - a.ph;
      const int t = x_voff + (n * a.C * HW + rbase * a.W) * 2;
#pragma unroll
      for (int it = 0; it < NX; ++it) {
        const bool ok = (unsigned)(x_row[it] + rbase) < (unsigned)a.H;
        rx[sI][it] = BufLoad<V>::ld(xrr, ok ? t + it * 2 * TPO * V : (int)0x80000000u, 0);
      }
      return;
    }
    const int n = step / a.steps_per_img;
    const int rem = step - n * a.steps_per_img;
    // first row, first x column of the step (whole rows: one segment at 0)
    const int pb = SEG ? rem / a.nseg : rem;
    const int p0 = pb * G, v0s = SEG ? (rem - pb * a.nseg) * a.XV : 0;
    // byte offsets of this step's image / first row (G divides P: all G dY rows exist)
    const int dys = dy_base_g + (n * a.O * PQ + p0 * a.Q) * 2;
    const int xso = x_base_g + (n * a.C * HW + (p0 - a.ph) * a.W) * 2;
    const int jmin = a.ph - p0, jmax = a.H + a.ph - p0;  // x rows j in [jmin, jmax) exist
    const int dc_org = v0s - a.HL;                       // dY column of run element 0
    int g = dg0, col = dc0;
#pragma unroll
    for (int it = 0; it < ND; ++it) {
      const int cg = SEG ? dc_org + col : col;  // a V-chunk is all inside [0, Q) or all outside
      const bool ok = dy_own_ok && sub + TPO * it < dy_chunks && (!SEG || (cg >= 0 && cg < a.Q));
      rdy[sI][it] = BufLoad<V>::ld(dyr, ok ? dys + (g * a.Q + cg) * 2 : (int)0x80000000u, 0);
      col += a.cadv;
      const int wrap = col >= a.RL;
      col -= wrap ? a.RL : 0;
      g += a.dadv + wrap;
    }
    int j = xj0;
    col = xc0;
#pragma unroll
    for (int it = 0; it < NX; ++it) {
      const int cg = SEG ? v0s + col : col;
      const bool ok = x_own_ok && sub + TPO * it < x_chunks && j >= jmin && j < jmax && (!SEG || cg < a.W);
      rx[sI][it] = BufLoad<V>::ld(xrr, ok ? xso + (j * a.W + cg) * 2 : (int)0x80000000u, 0);
      col += a.xcadv;
      const int wrap = col >= a.XL;
      col -= wrap ? a.XL : 0;
      j += a.xadv + wrap;
    }
  };
  auto sstore = [&](auto SET, int st) {
    constexpr int sI = decltype(SET)::value;
    if constexpr (!SEG) {
      uint16_t* base = smem + st * stage;
#pragma unroll
      for (int it = 0; it < ND; ++it) *reinterpret_cast<VT*>(base + d_lds[it]) = rdy[sI][it];
#pragma unroll
      for (int it = 0; it < NX; ++it) *reinterpret_cast<VT*>(base + x_lds[it]) = rx[sI][it];
      return;
    }
    // dY run element 0 (column v0s - HL) lands 8 - HL elements into the row's
    // slot, so column v0s is always at slot + 8
    uint16_t* d = DYS(st) + own * OS + (8 - a.HL);
    uint16_t* xs = XS(st) + own * CS;
    uint16_t* sink = smem + st * stage + dy_elems + x_elems;  // the stage's sink
    int g = dg0, col = dc0;
#pragma unroll
    for (int it = 0; it < ND; ++it) {
      uint16_t* dst = sub + TPO * it < dy_chunks ? d + g * DP + col : sink;
      *reinterpret_cast<VT*>(dst) = rdy[sI][it];
      col += a.cadv;
      const int wrap = col >= a.RL;
      col -= wrap ? a.RL : 0;
      g += a.dadv + wrap;
    }
    int j = xj0;
    col = xc0;
#pragma unroll
    for (int it = 0; it < NX; ++it) {
      uint16_t* dst = sub + TPO * it < x_chunks ? xs + j * XP + col : sink;
      *reinterpret_cast<VT*>(dst) = rx[sI][it];
      col += a.xcadv;
      const int wrap = col >= a.XL;
      col -= wrap ? a.XL : 0;
      j += a.xadv + wrap;
    }
  };

  f32x16 acc[RS];
  auto zero_acc = [&]() {
#pragma unroll
    for (int t = 0; t < RS; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[t][v] = 0.f;
  };
  if (!PC) zero_acc();
  float dbias = 0.f;
  const bool do_bias = a.dbias_part != nullptr && tile_c == 0;

  const int XV = a.XV;
  const int nchunk = G * (XV >> 3);  // even by construction
  const int grp = lane >> 5, rl = lane & 31;

  // Fragments of one 16-position step: the three aligned dY chunks around v0
  // (the dY windows of the three s taps) and the x chunk of each tap row r.
  struct Frag {
    u32x4w cm, cz, cp, x[R];
  };
  auto compute = [&](int st) {
    const uint16_t* dl = DYS(st) + (wo + rl) * OS + 8;
    const uint16_t* xl = XS(st) + (wc + rl) * CS;
    // this lane group's chunk t = kk + grp as (row g, column v0); branch-free
    // advance by 16 positions (XV is a multiple of 8, so at most two wraps)
    int g = 0, v0 = grp * 8;
    auto wrap = [&]() {
      const int w1 = v0 >= XV;
      v0 -= w1 ? XV : 0;
      g += w1;
      const int w2 = v0 >= XV;
      v0 -= w2 ? XV : 0;
      g += w2;
    };
    wrap();
    auto load = [&](Frag& f) {
      const uint16_t* dr = dl + g * DP + v0;
      const uint16_t* xr = xl + g * XP + v0;
      f.cm = *reinterpret_cast<const u32x4w*>(dr - 8);
      f.cz = *reinterpret_cast<const u32x4w*>(dr);
      f.cp = *reinterpret_cast<const u32x4w*>(dr + 8);
#pragma unroll
      for (int r = 0; r < R; ++r) f.x[r] = *reinterpret_cast<const u32x4w*>(xr + r * XP);
    };
    auto mma = [&](const Frag& f) {
      // dY windows for s = 0..2: start v0 + PW - s relative to the aligned chunk at v0
      bf16x8 af[S];
      af[0] = __builtin_bit_cast(bf16x8, window8<8 + PW>(f.cm, f.cz, f.cp));
      af[1] = __builtin_bit_cast(bf16x8, window8<7 + PW>(f.cm, f.cz, f.cp));
      af[2] = __builtin_bit_cast(bf16x8, window8<6 + PW>(f.cm, f.cz, f.cp));
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const bf16x8 bx = __builtin_bit_cast(bf16x8, f.x[r]);
#pragma unroll
        for (int s = 0; s < S; ++s)
          acc[r * S + s] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s], bx, acc[r * S + s], 0, 0, 0);
      }
    };
    // software pipeline: the LDS reads of step kk+1 are issued before the MFMAs
    // of step kk (the last prefetch re-reads the final step: harmless)
    const int nkk = nchunk >> 1;  // even number of chunks: nkk >= 1
    Frag fa, fb;
    if constexpr (KQ) {
      // this wave's MFMA steps kk = wave, wave + 4, ... < nkk: 64 positions
      // apart, i.e. dg rows + dv columns with at most one carry
      const int dg = 64 / XV, dv = 64 - dg * XV;
      auto step4 = [&]() {
        v0 += dv;
        g += dg;
        const int w1 = v0 >= XV;
        v0 -= w1 ? XV : 0;
        g += w1;
      };
      v0 += wave * 16;
      while (v0 >= XV) {  // at most 48 / 8 iterations, once per stage
        v0 -= XV;
        ++g;
      }
      const int nmy = (nkk - wave + 3) >> 2;  // wave-uniform, >= 0
      if (nmy > 0) {
        load(fa);
        int kk = 0;
        for (; kk + 2 <= nmy; kk += 2) {
          step4();
          load(fb);
          mma(fa);
          if (kk + 2 < nmy) step4();
          load(fa);
          mma(fb);
        }
        if (kk < nmy) mma(fa);
      }
    } else {
    load(fa);
    int kk = 0;
    for (; kk + 2 <= nkk; kk += 2) {
      v0 += 16;
      wrap();
      load(fb);
      mma(fa);
      if (kk + 2 < nkk) {
        v0 += 16;
        wrap();
      }
      load(fa);
      mma(fb);
    }
    if (kk < nkk) mma(fa);
    }
    if (do_bias) {
      // thread t sums quarter (t % 4) of the columns [8, 8 + BW) of every dY row
      // slot of o = t / 4: the step's own dY columns (past Q they hold zeros;
      // the halo columns of a segment belong to its neighbours)
      const uint16_t* drow = DYS(st) + own * OS + 8;
      const int q4 = a.BW / TPO, beg = sub * q4;
      for (int gg = 0; gg < G; ++gg)
        for (int k = beg; k < beg + q4; ++k) dbias += bf16_to_f32(drow[gg * DP + k]);
    }
  };

  __syncthreads();
  if constexpr (PC) {
    // One barrier per step on both sides.  Step ks is multiplied from LDS
    // buffer ks & 1 while the producers store step ks+1 into the other buffer
    // (read by the consumers before the previous barrier) and load later steps.
    if (producer) {
      if (nsteps > 0) {
        gload(I0{}, step_b);
        if (DEPTH == 2 && nsteps > 1) gload(I1{}, step_b + 1);
        __builtin_amdgcn_sched_barrier(0);
        sstore(I0{}, 0);
        if (DEPTH == 1 && nsteps > 1) gload(I0{}, step_b + 1);
        if (DEPTH == 2 && nsteps > 2) gload(I0{}, step_b + 2);
      }
      __syncthreads();
      for (int ks = 0; ks < nsteps; ks += 2) {
        // odd step ks+1 -> buffer 1 (register set 1 with two sets)
        if (ks + 1 < nsteps) sstore(I1{}, 1);
        if (DEPTH == 2 && ks + 3 < nsteps) gload(I1{}, step_b + ks + 3);
        if (DEPTH == 1 && ks + 2 < nsteps) gload(I0{}, step_b + ks + 2);
        __syncthreads();
        if (ks + 1 >= nsteps) break;
        // even step ks+2 -> buffer 0 (register set 0)
        if (ks + 2 < nsteps) sstore(I0{}, 0);
        if (DEPTH == 2 && ks + 4 < nsteps) gload(I0{}, step_b + ks + 4);
        if (DEPTH == 1 && ks + 3 < nsteps) gload(I0{}, step_b + ks + 3);
        __syncthreads();
      }
      if constexpr (!KQ) return;  // KQ: the producers take part in the epilogue's barriers
    } else {
      zero_acc();
      __syncthreads();
      for (int ks = 0; ks < nsteps; ++ks) {
        compute(ks & 1);
        __syncthreads();
      }
    }
  } else if constexpr (DEPTH == 2) {
    // invariant at an even ks: LDS buffer 0 holds step ks, register set 1
    // step ks+1 (in flight), set 0 is free; the steady-state loads are
    // unconditional so that each wait covers only the older set
    if (nsteps > 0) {
      gload(I0{}, step_b);
      if (nsteps > 1) gload(I1{}, step_b + 1);
      __builtin_amdgcn_sched_barrier(0);
      sstore(I0{}, 0);
    }
    __syncthreads();
    int ks = 0;
    for (; ks + 3 < nsteps; ks += 2) {
      gload(I0{}, step_b + ks + 2);
      __builtin_amdgcn_sched_barrier(0);
      compute(0);
      __builtin_amdgcn_sched_barrier(0);
      sstore(I1{}, 1);
      __syncthreads();
      gload(I1{}, step_b + ks + 3);
      __builtin_amdgcn_sched_barrier(0);
      compute(1);
      __builtin_amdgcn_sched_barrier(0);
      sstore(I0{}, 0);
      __syncthreads();
    }
    const int rem = nsteps - ks;  // 0 (no steps), 1, 2 or 3
    if (rem == 3) gload(I0{}, step_b + ks + 2);
    __builtin_amdgcn_sched_barrier(0);
    if (rem >= 1) compute(0);
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
  } else {
    if (nsteps > 0) {
      gload(I0{}, step_b);
      __builtin_amdgcn_sched_barrier(0);
      sstore(I0{}, 0);
    }
    __syncthreads();
    // steady state: the next step's loads are issued before this step's MFMAs
    // (sched_barrier keeps the compiler from sinking them to their use)
    for (int ks = 0; ks + 1 < nsteps; ++ks) {
      gload(I0{}, step_b + ks + 1);
      __builtin_amdgcn_sched_barrier(0);
      compute(ks & 1);
      __builtin_amdgcn_sched_barrier(0);
      sstore(I0{}, (ks + 1) & 1);
      __syncthreads();
    }
    if (nsteps > 0) compute((nsteps - 1) & 1);
  }
#undef DYS
#undef XS

  if constexpr (KQ) {
    // The four consumer waves hold partial sums of the same 32 x 32 x 9 tile.
    // Each writes its accumulators to LDS ([wave][tap][j][lane][4] floats,
    // 36 KB per wave; every stage has been read by now), then all 512 threads
    // add the four copies in wave order, 16 bytes at a time, and store the
    // block's partial tile in that same [tap][j][lane][4] layout.
    float4* red = reinterpret_cast<float4*>(smem);
    constexpr int Q4 = RS * 4 * 64;  // float4 units per wave copy
    if (!producer) {
#pragma unroll
      for (int t = 0; t < RS; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          red[(wave * RS + t) * 256 + j * 64 + lane] =
              float4{acc[t][4 * j], acc[t][4 * j + 1], acc[t][4 * j + 2], acc[t][4 * j + 3]};
    }
    __syncthreads();
    float4* pb = reinterpret_cast<float4*>(a.part) + ((long)split * a.tiles_o * a.tiles_c + tile) * Q4;
    for (int q = threadIdx.x; q < Q4; q += 512) {
      const float4 u0 = red[q], u1 = red[Q4 + q], u2 = red[2 * Q4 + q], u3 = red[3 * Q4 + q];
      pb[q] = float4{((u0.x + u1.x) + u2.x) + u3.x, ((u0.y + u1.y) + u2.y) + u3.y,
                     ((u0.z + u1.z) + u2.z) + u3.z, ((u0.w + u1.w) + u2.w) + u3.w};
    }
    if (producer) return;
  } else {
    float* pb = a.part + ((((long)split * a.tiles_o * a.tiles_c + tile) * 4 + wave) * RS) * 1024 + lane * 4;
#pragma unroll
    for (int t = 0; t < RS; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float4 u;
        u.x = acc[t][4 * j];
        u.y = acc[t][4 * j + 1];
        u.z = acc[t][4 * j + 2];
        u.w = acc[t][4 * j + 3];
        *reinterpret_cast<float4*>(pb + (t * 4 + j) * 256) = u;
      }
  }
  if (do_bias && !producer) {
    // combine the 4 quarter sums of each o (adjacent lanes)
    dbias += __shfl_xor(dbias, 1, 64);
    dbias += __shfl_xor(dbias, 2, 64);
    if constexpr (TPO == 8) dbias += __shfl_xor(dbias, 4, 64);
    const int o = o0 + own;
    if (sub == 0 && o < a.O) a.dbias_part[(long)split * a.O + o] = dbias;
  }
}

// dW[o][c][tap] = sum_z part[z][tap][o][c], bf16 out, in a fixed summation
// order (reduce_splits_block), so the result does not depend on timing.
// Blocks [0, nbw) reduce the dW partials, the rest the bias partials [split][O].
__global__ __launch_bounds__(256) void wgrad_reduce_bf16_kernel(const float* __restrict__ part, int splits,
                                                                int RS, int O, int C, uint16_t* __restrict__ dw,
                                                                const float* __restrict__ bpart,
                                                                uint16_t* __restrict__ db, int nbw) {
  if ((int)blockIdx.x < nbw) {
    // partials are [split][tap][O][C]; dW is OIHW
    reduce_splits_block(part, splits, (long)RS * O * C, [&](long i, float s) {
      const int c = (int)(i % C);
      const long t = i / C;
      const int o = (int)(t % O);
      const int tap = (int)(t / O);
      dw[((long)o * C + c) * RS + tap] = f32_to_bf16(s);
    }, (int)blockIdx.x, nbw);
  } else {
    reduce_splits_block(bpart, splits, (long)O, [&](long i, float s) { db[i] = f32_to_bf16(s); },
                        (int)blockIdx.x - nbw, (int)gridDim.x - nbw);
  }
}

// The same reduction read as float4 quads in split groups (many splits, few
// outputs: the few-channel kernel's 512 slabs), for R*S*O*C % 4 == 0 and
// O % 4 == 0 with 16-byte aligned slabs; the same fixed order for every run.
__global__ __launch_bounds__(256) void wgrad_reduce_vec4_bf16_kernel(const float* __restrict__ part, int splits,
                                                                     int RS, int O, int C, uint16_t* __restrict__ dw,
                                                                     const float* __restrict__ bpart,
                                                                     uint16_t* __restrict__ db, int nbw, int lg_g) {
  if ((int)blockIdx.x < nbw) {
    reduce_splits_vec4_block(part, splits, (long)RS * O * C, lg_g, [&](long i, float s) {
      const int c = (int)(i % C);
      const long t = i / C;
      const int o = (int)(t % O);
      const int tap = (int)(t / O);
      dw[((long)o * C + c) * RS + tap] = f32_to_bf16(s);
    }, (int)blockIdx.x, nbw);
  } else {
    reduce_splits_vec4_block(bpart, splits, (long)O, lg_g, [&](long i, float s) { db[i] = f32_to_bf16(s); },
                             (int)blockIdx.x - nbw, (int)gridDim.x - nbw);
  }
}

// The same for partials in the row kernel's accumulator layout (see the top of
// this file): element i of a split is ((((tile * 4 + wave) * RS + tap) * 4 + j)
// * 64 + lane) * 4 + k, i.e. dW[o][c][tap] with
//   o = o-tile * 64 + (wave / 2) * 32 + 8 j + 4 (lane / 32) + k,
//   c = c-tile * 64 + (wave % 2) * 32 + lane % 32   (tile = c-tile * tiles_o + o-tile);
// in the K-quarter form (kq) one 32 x 32 tile per block, no wave index:
//   o = o-tile * 32 + 8 j + 4 (lane / 32) + k,  c = c-tile * 32 + lane % 32.
__global__ __launch_bounds__(256) void wgrad_reduce_frag_bf16_kernel(const float* __restrict__ part, int splits,
                                                                     int RS, int tiles_o, int O, int C,
                                                                     uint16_t* __restrict__ dw,
                                                                     const float* __restrict__ bpart,
                                                                     uint16_t* __restrict__ db, int nbw, long total,
                                                                     int kq) {
  if ((int)blockIdx.x < nbw) {
    reduce_splits_block(part, splits, total, [&](long i, float s) {
      const int k = (int)(i & 3), lane = (int)((i >> 2) & 63), j = (int)((i >> 8) & 3);
      const long rest = i >> 10;
      const int tap = (int)(rest % RS);
      const long tw = rest / RS;
      int o, c;
      if (kq) {  // one 32 x 32 wave tile per block tile
        o = (int)(tw % tiles_o) * 32 + 8 * j + 4 * (lane >> 5) + k;
        c = (int)(tw / tiles_o) * 32 + (lane & 31);
      } else {
        const int wave = (int)(tw & 3);
        const long tile = tw >> 2;
        o = (int)(tile % tiles_o) * 64 + (wave >> 1) * 32 + 8 * j + 4 * (lane >> 5) + k;
        c = (int)(tile / tiles_o) * 64 + (wave & 1) * 32 + (lane & 31);
      }
      if (o < O && c < C) dw[((long)o * C + c) * RS + tap] = f32_to_bf16(s);
    }, (int)blockIdx.x, nbw);
  } else {
    reduce_splits_block(bpart, splits, (long)O, [&](long i, float s) { db[i] = f32_to_bf16(s); },
                        (int)blockIdx.x - nbw, (int)gridDim.x - nbw);
  }
}

// ---------------------------------------------------------------- few input channels
// Weight gradient for C <= 16 input channels (e.g. a first layer on RGB input),
// where a 64-wide channel tile would be mostly empty.  v_mfma_f32_16x16x32_bf16:
// D[o][c] (16 x 16) per tap, K = 32 x columns v of one output row p:
//   A[o][k] = dY[o][p][v + pw - s]   (lane: o = lane % 16, k = 8 * (lane / 16) ..)
//   B[k][c] = x[c][p + r - ph][v]    (lane: c = lane % 16, same k)
// Operands come straight from global memory (no LDS): each lane loads the
// aligned 8-column chunk v of its dY row -- its neighbours' chunks v-8 and v+8
// come from the lanes 16 below and above (ds_bpermute), the wave's outer ones
// from one more load -- (the windows of the S taps are funnel shifts of these)
// and the chunk v of its x channel in the R rows.
// Wave w of a block owns o0 + 16w .. +16 and walks the block's range of K steps
// (n, 32-column chunk, p), p fastest, with the next step's loads in flight; a
// step of the same chunk keeps R - 1 x rows of the previous one in registers.  Partials:
// [split][tap][O][C] and [split][O] for the bias, reduced like the row kernel's.
// af[i] = the 8 bf16 starting START - i elements into (c0, c1, c2), i < NW
template <int START, int NW>
struct DyWindows {
  __device__ static void run(bf16x8* af, const u32x4w& c0, const u32x4w& c1, const u32x4w& c2) {
    af[0] = __builtin_bit_cast(bf16x8, window8<START>(c0, c1, c2));
    DyWindows<START - 1, NW - 1>::run(af + 1, c0, c1, c2);
  }
};
template <int START>
struct DyWindows<START, 0> {
  __device__ static void run(bf16x8*, const u32x4w&, const u32x4w&, const u32x4w&) {}
};

struct SmallcArgs {
  const uint16_t* dy;  // [N][O][P][Q]
  const uint16_t* x;   // [N][C][H][W]
  float* part;         // [splits][RS][O][C]
  float* dbias_part;   // [splits][O] or nullptr
  int N, C, H, W, O, P, Q, ph;
  int nq;              // 32-column chunks per row: ceil(max(W, Q) / 32)
  int total_steps;     // N * P * nq
  int steps_per_split;
  int tiles_o;
  int dy_bytes, x_bytes;
};

template <int R, int S, int PW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void wgrad_smallc_bf16_kernel(SmallcArgs a) {
  static_assert(PW <= 2 && S - 1 - PW <= 2, "dY windows reach at most 2 columns either side");
  constexpr int RS = R * S;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile_o = blockIdx.x % a.tiles_o, split = blockIdx.x / a.tiles_o;
  const int ob = tile_o * 64 + wave * 16;  // the wave's first o
  const int kg = lane >> 4, li = lane & 15;
  const int o = ob + li, c = li;           // A row / B column of this lane
  const bool o_ok = o < a.O, c_ok = c < a.C;
  const int PQ = a.P * a.Q, HW = a.H * a.W;
  const __amdgpu_buffer_rsrc_t dyr = __builtin_amdgcn_make_buffer_rsrc((void*)a.dy, (short)0, a.dy_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t xrr = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.x_bytes, 0x00020000);
  const int OOR = (int)0x80000000u;

  const int step_b = split * a.steps_per_split;
  const int step_e = min(a.total_steps, step_b + a.steps_per_split);
  const int nsteps = step_e - step_b;  // >= 1 (splits are sized so)

  // cz: this lane's dY chunk (columns v .. v+7); ce: the chunk past the
  // wave's 32 columns on its side (v - 8 for kg = 0, v + 8 for kg = 3, zeros
  // elsewhere) -- the other lanes take their neighbours' cz at compute time
  struct Ops {
    u32x4w ce, cz, x[R];
  };
  // position of a step: (n, column chunk, p), p fastest, advanced
  // incrementally: consecutive steps of a chunk share R - 1 of their x rows
  int n, p, qc;
  {
    const int PN = a.P * a.nq;
    n = step_b / PN;
    const int rem = step_b - n * PN;
    qc = rem / a.P;
    p = rem - qc * a.P;
  }
  auto xrow_ld = [&](int r) {
    const int v = qc * 32 + kg * 8;
    const int h = p - a.ph + r;
    return BufLoad<8>::ld(xrr, c_ok && v < a.W && h >= 0 && h < a.H ? ((n * a.C + c) * HW + h * a.W + v) * 2 : OOR,
                          0);
  };
  auto load_dy = [&](Ops& f) {
    const int v = qc * 32 + kg * 8;  // this lane's 8 x columns v .. v+7
    const int drow = o_ok ? ((n * a.O + o) * PQ + p * a.Q) * 2 : 0;
    const int ve = kg == 0 ? v - 8 : v + 8;
    const bool edge = kg == 0 || kg == 3;
    f.cz = BufLoad<8>::ld(dyr, o_ok && v < a.Q ? drow + v * 2 : OOR, 0);
    f.ce = BufLoad<8>::ld(dyr, edge && o_ok && ve >= 0 && ve < a.Q ? drow + ve * 2 : OOR, 0);
  };
  auto load = [&](Ops& f) {
    load_dy(f);
#pragma unroll
    for (int r = 0; r < R; ++r) f.x[r] = xrow_ld(r);
  };
  // the step after prev's: within a chunk, x rows 1.. of prev are this step's
  // rows 0.. and only the last row is loaded (when the position did not move,
  // the final prefetch, the rows are never used)
  auto load_next = [&](Ops& f, const Ops& prev) {
    if (p == 0) {
      load(f);
    } else {
      load_dy(f);
#pragma unroll
      for (int r = 0; r + 1 < R; ++r) f.x[r] = prev.x[r + 1];
      f.x[R - 1] = xrow_ld(R - 1);
    }
  };
  auto advance = [&]() {
    ++p;
    const int w1 = p == a.P;
    p = w1 ? 0 : p;
    qc += w1;
    const int w2 = qc == a.nq;
    qc = w2 ? 0 : qc;
    n += w2;
  };

  f32x4 acc[RS];
#pragma unroll
  for (int t = 0; t < RS; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float bsum = 0.f;
  const bool do_bias = a.dbias_part != nullptr;

  auto compute = [&](const Ops& f) {
    // dY columns v + PW - s: window start 8 + PW - s in (cm, cz, cp); cm and
    // cp are the cz of the lanes 16 below / above (same o, the next 8 columns)
    u32x4w cm, cp;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = (uint32_t)__shfl((int)f.cz[i], lane - 16, 64);
      const uint32_t hi = (uint32_t)__shfl((int)f.cz[i], lane + 16, 64);
      cm[i] = kg == 0 ? f.ce[i] : lo;
      cp[i] = kg == 3 ? f.ce[i] : hi;
    }
    bf16x8 af[S];
    DyWindows<8 + PW, S>::run(af, cm, f.cz, cp);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const bf16x8 bx = __builtin_bit_cast(bf16x8, f.x[r]);
#pragma unroll
      for (int s = 0; s < S; ++s)
        acc[r * S + s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[s], bx, acc[r * S + s], 0, 0, 0);
    }
    if (do_bias) {
      // every dY chunk (row p, columns v .. v+7) is some step's cz exactly once
#pragma unroll
      for (int i = 0; i < 4; ++i)
        bsum += __uint_as_float(f.cz[i] << 16) + __uint_as_float(f.cz[i] & 0xffff0000u);
    }
  };

  // two operand sets: the loads of step k+1 are issued before the MFMAs of
  // step k; the last prefetch re-reads the final step (always in range)
  Ops fa, fb;
  load(fa);
  int k = 0;
  for (; k + 2 <= nsteps; k += 2) {
    advance();
    load_next(fb, fa);
    __builtin_amdgcn_sched_barrier(0);
    compute(fa);
    __builtin_amdgcn_sched_barrier(0);
    if (k + 2 < nsteps) advance();
    load_next(fa, fb);
    __builtin_amdgcn_sched_barrier(0);
    compute(fb);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (k < nsteps) compute(fa);

  // partials: lane holds D[o = ob + 4*kg + j][c = li]
#pragma unroll
  for (int t = 0; t < RS; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int oo = ob + kg * 4 + j;
      if (oo < a.O && c_ok) a.part[(((long)split * RS + t) * a.O + oo) * a.C + c] = acc[t][j];
    }
  if (do_bias) {
    bsum += __shfl_xor(bsum, 16, 64);
    bsum += __shfl_xor(bsum, 32, 64);
    if (kg == 0 && o_ok) a.dbias_part[(long)split * a.O + o] = bsum;
  }
}

// The same weight gradient for C * S <= 16 (an RGB 5x5 or a few-channel 3x3
// layer) with the MFMA's 16 B columns holding (c, s) = c * S + s instead of the
// channels alone: per row r one v_mfma_f32_16x16x32_bf16 covers every
// (channel, column tap) -- R MFMAs per K step instead of R * S with 13 of 16
// columns empty.  Operands: A = the lane's aligned 8-column dY chunk (o = lane %
// 16, columns v .. v+7 of the step's output row; no shifted windows, so no
// neighbour chunks of dY); B = for column j = (c, s) the 8 x values of channel c,
// input row p - ph + r, starting at column v + s - PW: a lane window taken at a
// lane-dependent offset (8 + s - PW elements) out of its channel's chunks v - 8,
// v, v + 8 (the outer ones from the lanes 16 below / above, or one more load at
// the wave's edges).  Rows walk as in wgrad_smallc_bf16_kernel (p fastest): a
// step computes the window of its one new x row and keeps the other R - 1.
// Partials: the same [split][tap][O][C] and [split][O] as that kernel.
template <int R, int S, int PW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 4))) void wgrad_smallc_cs_bf16_kernel(
    SmallcArgs a) {
  static_assert(PW <= 2 && S - 1 - PW <= 2, "x windows reach at most 2 columns either side");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile_o = blockIdx.x % a.tiles_o, split = blockIdx.x / a.tiles_o;
  const int ob = tile_o * 64 + wave * 16;  // the wave's first o
  const int kg = lane >> 4, li = lane & 15;
  const int o = ob + li;                   // A row of this lane
  const int c = li / S, s = li - (li / S) * S;  // B column (c, s) of this lane
  const bool o_ok = o < a.O, c_ok = li < a.C * S;
  const int PQ = a.P * a.Q, HW = a.H * a.W;
  const __amdgpu_buffer_rsrc_t dyr = __builtin_amdgcn_make_buffer_rsrc((void*)a.dy, (short)0, a.dy_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t xrr = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.x_bytes, 0x00020000);
  const int OOR = (int)0x80000000u;
  // window start (elements) in the lane's 24 x columns v - 8 .. v + 15: the
  // window's dwords start at dword 3 + t (t = e / 2 - 3 in 0..3), shifted by a
  // half dword when e is odd; selections as bit masks (branch-free: the lanes
  // of a wave take different t)
  const int e = 8 + s - PW, t3 = (e >> 1) - 3;
  const uint32_t m1 = (t3 & 1) ? ~0u : 0u, m2 = (t3 & 2) ? ~0u : 0u, modd = (e & 1) ? ~0u : 0u;

  const int step_b = split * a.steps_per_split;
  const int step_e = min(a.total_steps, step_b + a.steps_per_split);
  const int nsteps = step_e - step_b;  // >= 1 (splits are sized so)

  // operands of a step: the dY chunk, and the x chunk (+ the wave-edge chunk)
  // of each x row it has to load (all R at a chunk's first row, else the last)
  struct Ops {
    u32x4w dz, xz[R], xe[R];
  };
  int n, p, qc;
  {
    const int PN = a.P * a.nq;
    n = step_b / PN;
    const int rem = step_b - n * PN;
    qc = rem / a.P;
    p = rem - qc * a.P;
  }
  auto xrow_ld = [&](Ops& f, int r, int slot) {
    const int v = qc * 32 + kg * 8, ve = kg == 0 ? v - 8 : v + 8;
    const bool edge = kg == 0 || kg == 3;
    const int h = p - a.ph + r;
    const bool hok = c_ok && h >= 0 && h < a.H;
    const int rb = ((n * a.C + c) * HW + h * a.W) * 2;
    f.xz[slot] = BufLoad<8>::ld(xrr, hok && v < a.W ? rb + v * 2 : OOR, 0);
    f.xe[slot] = BufLoad<8>::ld(xrr, hok && edge && ve >= 0 && ve < a.W ? rb + ve * 2 : OOR, 0);
  };
  // all: load every x row (a chunk's first row, or a split's first step)
  auto load = [&](Ops& f, bool all) {
    const int v = qc * 32 + kg * 8;
    f.dz = BufLoad<8>::ld(dyr, o_ok && v < a.Q ? ((n * a.O + o) * PQ + p * a.Q + v) * 2 : OOR, 0);
    if (all) {
#pragma unroll
      for (int r = 0; r < R; ++r) xrow_ld(f, r, r);
    } else {
      xrow_ld(f, R - 1, R - 1);
    }
  };
  auto advance = [&]() {
    ++p;
    const int w1 = p == a.P;
    p = w1 ? 0 : p;
    qc += w1;
    const int w2 = qc == a.nq;
    qc = w2 ? 0 : qc;
    n += w2;
  };
  // the lane's window of one x row: 8 elements from offset e of (xm, xz, xp)
  auto window = [&](const u32x4w& xz, const u32x4w& xe) {
    uint32_t w[12];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = (uint32_t)__shfl((int)xz[i], lane - 16, 64);
      const uint32_t hi = (uint32_t)__shfl((int)xz[i], lane + 16, 64);
      w[i] = kg == 0 ? xe[i] : lo;
      w[4 + i] = xz[i];
      w[8 + i] = kg == 3 ? xe[i] : hi;
    }
    auto pick = [](uint32_t m, uint32_t a, uint32_t b) { return (a & m) | (b & ~m); };  // m ? a : b
    u32x4w out;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // dwords 3 + t3 + i and 4 + t3 + i
      const uint32_t d0 = pick(m2, pick(m1, w[6 + i], w[5 + i]), pick(m1, w[4 + i], w[3 + i]));
      const uint32_t d1 = pick(m2, pick(m1, w[7 + i], w[6 + i]), pick(m1, w[5 + i], w[4 + i]));
      out[i] = pick(modd, __builtin_amdgcn_alignbyte(d1, d0, 2), d0);
    }
    return out;
  };

  f32x4 acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  float bsum = 0.f;
  const bool do_bias = a.dbias_part != nullptr;
  u32x4w win[R];  // the windows of the step's R x rows (rows 0 .. R-2 carried over)

  // all: the step loaded every x row (all R windows new)
  auto compute = [&](const Ops& f, bool all) {
    if (all) {
#pragma unroll
      for (int r = 0; r < R; ++r) win[r] = window(f.xz[r], f.xe[r]);
    } else {
#pragma unroll
      for (int r = 0; r + 1 < R; ++r) win[r] = win[r + 1];
      win[R - 1] = window(f.xz[R - 1], f.xe[R - 1]);
    }
    const bf16x8 ad = __builtin_bit_cast(bf16x8, f.dz);
#pragma unroll
    for (int r = 0; r < R; ++r)
      acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ad, __builtin_bit_cast(bf16x8, win[r]), acc[r], 0, 0, 0);
    if (do_bias) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        bsum += __uint_as_float(f.dz[i] << 16) + __uint_as_float(f.dz[i] & 0xffff0000u);
    }
  };

  // two operand sets: the loads of step k+1 are issued before the MFMAs of
  // step k; the last prefetch re-reads the final step (always in range)
  Ops fa, fb;
  bool all_a = true, all_b;  // the split's first step has no carried windows
  load(fa, true);
  int k = 0;
  for (; k + 2 <= nsteps; k += 2) {
    advance();
    all_b = p == 0;
    load(fb, all_b);
    __builtin_amdgcn_sched_barrier(0);
    compute(fa, all_a);
    __builtin_amdgcn_sched_barrier(0);
    if (k + 2 < nsteps) advance();
    all_a = p == 0;
    load(fa, all_a);
    __builtin_amdgcn_sched_barrier(0);
    compute(fb, all_b);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (k < nsteps) compute(fa, all_a);

  // partials: lane holds D[o = ob + 4*kg + j][column li = (c, s)] for each row r
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int oo = ob + kg * 4 + j;
      if (oo < a.O && c_ok) a.part[(((long)split * R * S + r * S + s) * a.O + oo) * a.C + c] = acc[r][j];
    }
  if (do_bias) {
    bsum += __shfl_xor(bsum, 16, 64);
    bsum += __shfl_xor(bsum, 32, 64);
    if (kg == 0 && o_ok) a.dbias_part[(long)split * a.O + o] = bsum;
  }
}

namespace {

struct WgradPlan {
  WgradArgs a;
  int splits, nd, nx;
  size_t lds;
  int tiles_o, tiles_c;
  bool kq;  // 32 x 32 tiles, K quarters (partials: one wave tile per block)
};

// kq: whole rows only, 32 x 32 block tiles with the K quarters of the KQ form
// (false when the rows need column segments).
bool plan_wgrad(WgradPlan& pl, int N, int C, int H, int W, int O, int R, int S, int ph, int pw, bool kq = false) {
  WgradArgs& a = pl.a;
  const int TT = kq ? 32 : 64, TPO = 256 / TT;
  const int P = H + 2 * ph - R + 1, Q = W + 2 * pw - S + 1;
  if (P <= 0 || Q <= 0 || R != 3 || S != 3 || ph > 2 || pw > 2) return false;
  a.N = N; a.C = C; a.H = H; a.W = W; a.O = O; a.P = P; a.Q = Q; a.ph = ph; a.pw = pw;
  // vector width: divides Q and W (rows start at multiples of Q / W elements)
  a.V = 8;
  while (a.V > 1 && ((Q % a.V) || (W % a.V))) a.V >>= 1;
  if (a.V < 2) return false;

  // Whole rows if they fit (the largest row count G dividing P whose two LDS
  // stages fit in 160 KB), else column segments of 128, 64, 32 or 16 x columns
  // (dY loaded with 8 columns on either side), choosing the segment width and
  // G with the fewest loaded elements per output position.
  a.G = 0;
  const int wfull = (W + 7) / 8 * 8, span = std::max(W, Q);
  const int seg_w[] = {wfull, 128, 64, 32, 16};
  double best = 1e30;
  for (int si = 0; si < 5; ++si) {
    const int sw = seg_w[si];
    const bool whole = si == 0;
    if (!whole && (a.G != 0 && a.HL == 0)) break;  // whole rows fit
    if (!whole && sw >= wfull) continue;
    for (int g = P; g >= 1; --g) {
      if (P % g) continue;
      int xv = sw;
      if ((g * (xv / 8)) & 1) {
        if (!whole) continue;         // segment widths are fixed: need an even chunk count
        xv += 8;                      // whole rows: one zero chunk more
      }
      const int hl = whole ? 0 : 8;
      const int rl = whole ? Q : xv + 16, xl = whole ? W : xv;
      if (rl % a.V || xl % a.V) continue;
      const int dp = whole ? std::max(xv, (Q + 7) / 8 * 8) + 8 : xv + 16;
      int os = whole ? 8 + g * dp : g * dp;
      if (((os / 8) & 1) == 0) os += 8;  // odd number of 16-byte units: conflict-free
      int cs = (g + R - 1) * xv;
      if (((cs / 8) & 1) == 0) cs += 8;
      const size_t lds = 2 * ((size_t)(TT * os + TT * cs) + 8) * 2;  // + a 16-byte sink per stage
      const int nd = (g * (rl / a.V) + TPO - 1) / TPO, nx = ((g + R - 1) * (xl / a.V) + TPO - 1) / TPO;
      if (lds > 160 * 1024 || nd > 16 || nx > 16) continue;
      const double cost = double(g * rl + (g + R - 1) * xl) / double(g * xv);
      if (!whole && cost >= best) continue;
      best = cost;
      a.G = g;
      a.XV = xv;
      a.XP = xv;
      a.DP = dp;
      a.OS = os;
      a.CS = cs;
      a.HL = hl;
      a.RL = rl;
      a.XL = xl;
      a.BW = whole ? dp - 8 : xv;
      a.nseg = whole ? 1 : (span + xv - 1) / xv;
      pl.lds = lds;
      pl.nd = nd;
      pl.nx = nx;
      if (whole) break;  // largest G
    }
  }
  if (a.G == 0) return false;
  // K quarters: whole rows, and the MFMA steps of a K step (16 positions each)
  // dealt evenly over the four waves (measured: 14 steps -> 4,4,3,3 was slower
  // than the 64 x 64 form)
  if (kq && (a.nseg != 1 || a.HL != 0 || (a.G * a.XV / 16) % 4 != 0)) return false;
  if (kq) pl.lds = std::max<size_t>(pl.lds, (size_t)4 * R * S * 1024 * sizeof(float));  // the epilogue's sum
  a.cpr_dy = a.RL / a.V;
  a.cpr_x = a.XL / a.V;
  a.dadv = TPO * a.V / a.RL;
  a.cadv = TPO * a.V % a.RL;
  a.xadv = TPO * a.V / a.XL;
  a.xcadv = TPO * a.V % a.XL;
  a.steps_per_img = P / a.G * a.nseg;
  a.total_steps = N * a.steps_per_img;
  pl.kq = kq;
  pl.tiles_o = (O + TT - 1) / TT;
  pl.tiles_c = (C + TT - 1) / TT;
  const int tiles = pl.tiles_o * pl.tiles_c;
  // one wave of blocks over the 256 CUs (one block per CU: LDS-limited)
  int splits = std::max(1, std::min(a.total_steps, (256 + tiles - 1) / tiles));
  a.steps_per_split = (a.total_steps + splits - 1) / splits;
  pl.splits = (a.total_steps + a.steps_per_split - 1) / a.steps_per_split;
  a.tiles_o = pl.tiles_o;
  a.tiles_c = pl.tiles_c;
  a.splits = pl.splits;
  return true;
}

// Plan of the few-channel kernel: false if the shape is outside its envelope.
bool plan_smallc(SmallcArgs& a, int N, int C, int H, int W, int O, int R, int S, int ph, int pw) {
  const int P = H + 2 * ph - R + 1, Q = W + 2 * pw - S + 1;
  if (P <= 0 || Q <= 0 || C < 1 || C > 16 || (W % 8) || (Q % 8)) return false;
  if (!((R == 3 && S == 3) || (R == 5 && S == 5 && pw == 2))) return false;
  if (pw > 2 || S - 1 - pw > 2) return false;
  const long dyb = (long)N * O * P * Q * 2, xb = (long)N * C * H * W * 2;
  if (dyb >= (1L << 31) - 64 || xb >= (1L << 31) - 64) return false;
  a.N = N; a.C = C; a.H = H; a.W = W; a.O = O; a.P = P; a.Q = Q; a.ph = ph;
  a.nq = (std::max(W, Q) + 31) / 32;
  a.total_steps = N * P * a.nq;
  a.tiles_o = (O + 63) / 64;
  // about two blocks per CU (the per-channel kernel: ~190 VGPRs, two waves
  // per SIMD; the (channel, tap) kernel fits three, but 768 blocks measured
  // equal in its loop and 3 us slower in the reduction of their partials)
  const int splits = std::max(1, std::min(a.total_steps, (512 + a.tiles_o - 1) / a.tiles_o));
  a.steps_per_split = (a.total_steps + splits - 1) / splits;
  a.dy_bytes = (int)dyb;
  a.x_bytes = (int)xb;
  return true;
}

int smallc_splits(const SmallcArgs& a) { return (a.total_steps + a.steps_per_split - 1) / a.steps_per_split; }

int launch_smallc(const SmallcArgs& a, int R, int S, int pw, hipStream_t st) {
  const dim3 grid((unsigned)(a.tiles_o * smallc_splits(a)));
  if (a.C * S <= 16) {  // (channel, column tap) in the MFMA columns
    if (R == 5) {
      wgrad_smallc_cs_bf16_kernel<5, 5, 2><<<grid, 256, 0, st>>>(a);
    } else if (pw == 0) {
      wgrad_smallc_cs_bf16_kernel<3, 3, 0><<<grid, 256, 0, st>>>(a);
    } else if (pw == 1) {
      wgrad_smallc_cs_bf16_kernel<3, 3, 1><<<grid, 256, 0, st>>>(a);
    } else {
      wgrad_smallc_cs_bf16_kernel<3, 3, 2><<<grid, 256, 0, st>>>(a);
    }
    VH_LAUNCH_CHECK();
    return VH_OK;
  }
  if (R == 5) {
    wgrad_smallc_bf16_kernel<5, 5, 2><<<grid, 256, 0, st>>>(a);
  } else if (pw == 0) {
    wgrad_smallc_bf16_kernel<3, 3, 0><<<grid, 256, 0, st>>>(a);
  } else if (pw == 1) {
    wgrad_smallc_bf16_kernel<3, 3, 1><<<grid, 256, 0, st>>>(a);
  } else {
    wgrad_smallc_bf16_kernel<3, 3, 2><<<grid, 256, 0, st>>>(a);
  }
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <int R, int S, int PW, int V, int ND, int NX, bool SEG, int DEPTH = 1, bool PC = false, bool KQ = false>
int launch_wgrad(const WgradPlan& pl, hipStream_t st) {
  auto kern = wgrad_rows_bf16_kernel<R, S, PW, V, ND, NX, SEG, DEPTH, PC, KQ>;
  VH_LDS_LIMIT_ONCE(kern);
  dim3 grid((unsigned)(pl.tiles_o * pl.tiles_c * pl.splits));
  kern<<<grid, PC ? 512 : 256, pl.lds, st>>>(pl.a);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

template <int PW, int V>
int launch_v(const WgradPlan& pl, hipStream_t st) {
  const int n = std::max(pl.nd, pl.nx);
  const bool seg = pl.a.nseg > 1 || pl.a.HL != 0;
  if (pl.kq) {  // whole rows, producer / consumer, K quarters
    if constexpr (V == 8) {
      if (pl.nd <= 8 && pl.nx <= 8) return launch_wgrad<3, 3, PW, V, 8, 8, false, 1, true, true>(pl, st);
      if (pl.nd <= 12 && pl.nx <= 12) return launch_wgrad<3, 3, PW, V, 12, 12, false, 1, true, true>(pl, st);
      if (pl.nd <= 16 && pl.nx <= 16) return launch_wgrad<3, 3, PW, V, 16, 16, false, 1, true, true>(pl, st);
    } else {
      if (pl.nd <= 16 && pl.nx <= 16) return launch_wgrad<3, 3, PW, V, 16, 16, false, 2, true, true>(pl, st);
    }
    return VH_ERR_UNSUPPORTED;
  }
  // two register sets when they fit (16-byte items: at most 6 + 6; 4- and
  // 8-byte items of whole rows: 16 + 16)
  // producer / consumer blocks for whole rows and for the 16-byte-item segment
  // form (below); whole rows (the producers' register sets: two
  // for 4- and 8-byte items, one closer-fitting set for 16-byte items)
  if (!seg) {
    if constexpr (V == 8) {
      if (pl.nd <= 8 && pl.nx <= 8) return launch_wgrad<3, 3, PW, V, 8, 8, false, 1, true>(pl, st);
      if (pl.nd <= 8 && pl.nx <= 12) return launch_wgrad<3, 3, PW, V, 8, 12, false, 1, true>(pl, st);
      if (pl.nd <= 12 && pl.nx <= 16) return launch_wgrad<3, 3, PW, V, 12, 16, false, 1, true>(pl, st);
      if (pl.nd <= 16 && pl.nx <= 16) return launch_wgrad<3, 3, PW, V, 16, 16, false, 1, true>(pl, st);
    } else {
      if (pl.nd <= 16 && pl.nx <= 16) return launch_wgrad<3, 3, PW, V, 16, 16, false, 2, true>(pl, st);
    }
  }
  if constexpr (V == 8) {
    if (pl.nd <= 6 && pl.nx <= 6)
      return seg ? launch_wgrad<3, 3, PW, V, 6, 6, true, 2, true>(pl, st)
                 : launch_wgrad<3, 3, PW, V, 6, 6, false, 2>(pl, st);
  } else {
    if (!seg && pl.nd <= 16 && pl.nx <= 16) return launch_wgrad<3, 3, PW, V, 16, 16, false, 2>(pl, st);
  }
  if (n <= 8) return seg ? launch_wgrad<3, 3, PW, V, 8, 8, true>(pl, st) : launch_wgrad<3, 3, PW, V, 8, 8, false>(pl, st);
  // whole rows: closer-fitting item counts (unused items still issue a load and a sink store)
  if (!seg && pl.nd <= 8 && pl.nx <= 12) return launch_wgrad<3, 3, PW, V, 8, 12, false>(pl, st);
  if (!seg && pl.nd <= 12 && pl.nx <= 16) return launch_wgrad<3, 3, PW, V, 12, 16, false>(pl, st);
  if (n <= 16)
    return seg ? launch_wgrad<3, 3, PW, V, 16, 16, true>(pl, st) : launch_wgrad<3, 3, PW, V, 16, 16, false>(pl, st);
  return VH_ERR_UNSUPPORTED;
}

// partials of the row kernel: [split][tile][4 waves][tap][1024]
size_t frag_part_bytes(const WgradPlan& pl, int RS) {
  return (size_t)pl.splits * pl.tiles_o * pl.tiles_c * (pl.kq ? 1 : 4) * RS * 1024 * sizeof(float);
}

template <int PW>
int launch_pw(const WgradPlan& pl, hipStream_t st) {
  return pl.a.V == 8 ? launch_v<PW, 8>(pl, st) : pl.a.V == 4 ? launch_v<PW, 4>(pl, st) : launch_v<PW, 2>(pl, st);
}

}  // namespace

// The K-quarter form (a quarter of the partial bytes) where it computes fewer
// padded rows / columns than 64 x 64 tiles (O or C not a multiple of 64), or
// where a K step spans at least 4 output rows; else the 64 x 64 form.
// Measured: with one output row per K step (256-wide rows) the K-quarter form
// stages 3 input rows per output row and was slower than 64 x 64 segments.
static bool plan_rows(WgradPlan& pl, int N, int C, int H, int W, int O, int R, int S, int ph, int pw) {
  WgradPlan kq;
  if (plan_wgrad(kq, N, C, H, W, O, R, S, ph, pw, true)) {
    const long pad64 = (long)((O + 63) / 64 * 64) * ((C + 63) / 64 * 64);
    const long pad32 = (long)((O + 31) / 32 * 32) * ((C + 31) / 32 * 32);
    if (pad32 < pad64 || kq.a.G >= 4) {
      pl = kq;
      return true;
    }
  }
  return plan_wgrad(pl, N, C, H, W, O, R, S, ph, pw, false);
}

size_t wgrad_rows_ws(int N, int C, int H, int W, int O, int R, int S, int ph, int pw, bool bias) {
  SmallcArgs sa;
  if (plan_smallc(sa, N, C, H, W, O, R, S, ph, pw)) {
    const int splits = smallc_splits(sa);
    size_t b = (size_t)splits * R * S * O * C * sizeof(float);
    if (bias) b = ((b + 255) & ~size_t(255)) + (size_t)splits * O * sizeof(float);
    return b;
  }
  WgradPlan pl;
  if (!plan_rows(pl, N, C, H, W, O, R, S, ph, pw)) return 0;
  size_t b = frag_part_bytes(pl, R * S);
  if (bias) b += (size_t)pl.splits * O * sizeof(float) + 256;
  return b;
}

int wgrad_rows_bf16(const void* dy, const void* x, void* dw, void* db, int N, int C, int H, int W, int O, int R,
                    int S, int ph, int pw, float* ws, size_t ws_bytes, hipStream_t st) {
  const size_t need = wgrad_rows_ws(N, C, H, W, O, R, S, ph, pw, db != nullptr);
  if (need == 0) return VH_ERR_UNSUPPORTED;
  if (need > ws_bytes) return set_error(VH_ERR_BAD_ARG, "wgrad workspace too small");
  SmallcArgs sa;
  if (plan_smallc(sa, N, C, H, W, O, R, S, ph, pw)) {
    const int splits = smallc_splits(sa);
    const size_t pbytes = (size_t)splits * R * S * O * C * sizeof(float);
    sa.dy = (const uint16_t*)dy;
    sa.x = (const uint16_t*)x;
    sa.part = ws;
    sa.dbias_part = db ? (float*)((char*)ws + ((pbytes + 255) & ~size_t(255))) : nullptr;
    VH_TRY_W(launch_smallc(sa, R, S, pw, st));
    const long total = (long)R * S * O * C;
    if (total % 4 == 0 && O % 4 == 0) {
      // slabs start 16-byte aligned (ws, and the bias slabs at a 256-byte offset)
      const int lg_g = reduce_vec4_lg_groups(splits);
      const int nbw = reduce_vec4_grid(total, lg_g), nbb = db ? reduce_vec4_grid(O, lg_g) : 0;
      wgrad_reduce_vec4_bf16_kernel<<<nbw + nbb, 256, 0, st>>>(ws, splits, R * S, O, C, (uint16_t*)dw,
                                                               sa.dbias_part, (uint16_t*)db, nbw, lg_g);
      VH_LAUNCH_CHECK();
      return VH_OK;
    }
    const int nbw = reduce_splits_grid(total), nbb = db ? reduce_splits_grid(O) : 0;
    wgrad_reduce_bf16_kernel<<<nbw + nbb, 256, 0, st>>>(ws, splits, R * S, O, C, (uint16_t*)dw, sa.dbias_part,
                                                        (uint16_t*)db, nbw);
    VH_LAUNCH_CHECK();
    return VH_OK;
  }
  WgradPlan pl;
  if (!plan_rows(pl, N, C, H, W, O, R, S, ph, pw)) return VH_ERR_UNSUPPORTED;
  {
    const long dyb = (long)N * O * pl.a.P * pl.a.Q * 2, xb = (long)N * C * H * W * 2;
    if (dyb >= (1L << 31) - 16 || xb >= (1L << 31) - 16) return VH_ERR_UNSUPPORTED;
    pl.a.dy_bytes = (int)dyb;
    pl.a.x_bytes = (int)xb;
  }
  pl.a.dy = (const uint16_t*)dy;
  pl.a.x = (const uint16_t*)x;
  pl.a.part = ws;
  const size_t pbytes = frag_part_bytes(pl, R * S);
  pl.a.dbias_part = db ? (float*)((char*)ws + ((pbytes + 255) & ~size_t(255))) : nullptr;
  int rc = pl.a.pw == 0 ? launch_pw<0>(pl, st) : pl.a.pw == 1 ? launch_pw<1>(pl, st) : launch_pw<2>(pl, st);
  if (rc) return rc;
  const long total = (long)(pbytes / sizeof(float) / pl.splits);
  const int nbw = reduce_splits_grid(total), nbb = db ? reduce_splits_grid(O) : 0;
  wgrad_reduce_frag_bf16_kernel<<<nbw + nbb, 256, 0, st>>>(ws, pl.splits, R * S, pl.tiles_o, O, C, (uint16_t*)dw,
                                                           pl.a.dbias_part, (uint16_t*)db, nbw, total, pl.kq ? 1 : 0);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

}  // namespace vh
