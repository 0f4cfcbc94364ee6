// vh_halo.hip -- bf16 implicit-GEMM convolution for stride-1 layers on NCHW
// tensors, gfx950 MFMA (v_mfma_f32_32x32x16_bf16).  Serves the forward pass
// and, with a flipped/transposed weight, the input gradient.
//
// GEMM view: rows = output channels o, columns = output positions m = (n,p,q)
// (flattened over the batch), K = (input channel c, tap r, tap s).
//
// A block owns BM output channels x BN consecutive positions.  For every group
// of 16 input channels it stages in LDS
//   * the weights  W[o][tap][c16]          (K-packed per (o, tap)), and
//   * the input "halo": every padded input row the BN positions touch, stored
//     channel-packed, cell = (ext row, padded column) -> 16 channels,
// then runs all R*S taps against that one copy of the input: tap (r,s) of
// position (n,p,q) is the cell (n*Hp + p + r, q + s), i.e. a fixed LDS address
// shift.  x is read from HBM once per block (plus the halo rows), with dword
// loads along rows that are transposed to channel-packed cells in registers.
//
// Each ext row holds two half-planes (channels 0-7, 8-15) side by side so that
// the 64 lanes of one fragment read walk consecutive 16-byte cells: lanes 0-31
// read plane 0, lanes 32-63 plane 1, each at consecutive positions / output
// channels.  A ds_read_b128 serves 16 lanes per cycle, lanes {0-3, 12-15,
// 20-27} and {4-11, 16-19, 28-31} (and the same sets + 32), which together
// read 16 positions spread over 28 consecutive ones: those are on distinct
// banks only if every row end (and image end) moves the cell index by a
// multiple of 16 cells, hence the row pitch Wp = TW (mod 16) and the per-image
// offset img_d.  Putting both half-planes in one row pitch is what makes the
// aligned pitch fit the fused form's stage (2 Wr + 15 cells a row instead of
// 2 (Wr + 15)).
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "vh_kernels.hpp"

namespace vh {

#define VH_TRY_HALO(expr)       \
  do {                          \
    int _s = (expr);            \
    if (_s != VH_OK) return _s; \
  } while (0)

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

struct HaloArgs {
  const uint16_t* x;     // [N][C][H][W]
  const uint16_t* wt;    // grouped [C/16][O][2*R*S+1][8] (last unit zero)
  const uint16_t* bias;  // [O] or nullptr
  uint16_t* y;           // [N][O][P][Q]
  int N, C, H, W, O, P, Q, ph, pw;
  // Column strips: the output is cut into nstrips strips of TW columns; strip j
  // of image n is "virtual image" n*nstrips + j of P x TW positions (positions
  // past Q are computed and dropped).  One strip (TW = Q) means whole rows.
  int TW, nstrips;
  int Hp;                // padded input rows: H + 2*ph
  int Wp;                // LDS cells per ext row, both half-planes: plane 0 at cells [0, Wr),
                         // plane 1 at [hoff, hoff + Wr) (Wr = TW + S - 1 + cs, even; Wp >= 2 Wr),
                         // = TW mod 16 where the LDS budget allows (conflict-free fragment reads)
  int hoff;              // cell offset of half-plane 1 within an ext row
  int img_d;             // extra cells per virtual image past the block's first: keeps the
                         // cell jump between images = 0 mod 16 (0 when Wp is not aligned)
  int xcells;            // x cells per LDS stage: rows_max * Wp + (images spanned - 1) * img_d
  int cs;                // cell of input column strip*TW - pw (0, or 1 for strips
                         // with pw odd: cell 0 then sits on an even input column)
  int lcol0, lcell0;     // first loaded column pair: input column strip*TW + lcol0
                         // goes to cell lcell0 (whole rows: 0 -> pw, padding
                         // cells zeroed once; strips: -pw-cs -> 0, all loaded)
  int npairs;            // column pairs loaded per ext row
  int M;                 // N*nstrips*P*TW virtual positions
  int rows_max;          // max ext rows any block needs
  int x_bytes;           // size of x in bytes (< 2^31: buffer-load range)
  int y_bytes;           // size of y in bytes (< 2^31)
  int w_bytes;           // size of wt in bytes
  int tiles_m, tiles_o;  // grid = tiles_m * tiles_o blocks
  int act;               // epilogue: 0 none, 1 ReLU, 2 zero where mask <= 0 (mask laid out like y)
  const uint16_t* mask;
  int stages;            // LDS stages (1 when there is a single channel group)
  int vec_epi;           // 1: whole rows, P*Q % 8 == 0 and 16-byte aligned y / mask:
                         // the epilogue transposes through LDS and stores 8 positions per lane
  int pair_epi;          // 1: Q even, 4-byte aligned y / mask: lane pairs exchange values and
                         // store two positions of one row per lane (no LDS)
  FastDiv fPQ, fQ;              // P*TW, TW
  FastDiv fW2, fRowsMax, fHp;   // item decomposition (Wp/2, rows_max, Hp)
  FastDiv fStrips;              // nstrips
};

// FMT: 32-row fragments per wave along the output channels (2: 64 o per wave;
// 1: 32, the tile for layers with at most 32 output channels)
template <int R, int S, int WM, int XI, int FMT = 2>
struct HaloCfg {
  static constexpr int RS = R * S;
  static constexpr int FM = FMT, FN = 2;          // 32x32 tiles per wave
  static constexpr int WN = 4 / WM;               // waves along positions
  static constexpr int BM = WM * FM * 32;
  static constexpr int BN = WN * FN * 32;
  static constexpr int WPU = 2 * RS + 1;          // units per output channel (odd: conflict-free reads)
  static constexpr int WUNITS = BM * WPU;         // 16-byte weight units per stage
  static constexpr int WITER = (WUNITS + 255) / 256;
  static constexpr int XITER = XI;                // x items per thread per stage (8 dwords each)
};

__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
  // low bf16 of a, low bf16 of b -> (a.lo | b.lo << 16)
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// LDS units (16 bytes) per stage of the fused form: two stages of 38.9 KB, two
// blocks per CU.
constexpr int kFusedStageUnits = 2432;

// The fused form as producer / consumer blocks (512 threads, four waves per SIMD).
#ifndef VH_HALO_PC
#define VH_HALO_PC 1
#endif
#define VH_HALO_FUSED_WPE (VH_HALO_PC ? 4 : 2)

// Fragment-read lookahead (in taps) of the producer / consumer form's consumers.
#ifndef VH_HALO_PC_LA
#define VH_HALO_PC_LA 1
#endif

// Grids of at least this many tiles (3x3, several channel groups) use one LDS
// stage and three blocks per CU.
#ifndef VH_HALO_WPE3_MIN_TILES
#define VH_HALO_WPE3_MIN_TILES 1024
#endif

// WPE = waves per SIMD the kernel is compiled for.  WPE 2: two LDS stages and
// (for narrow tiles) two register sets, two blocks per CU.  WPE 3: one LDS
// stage and one register set (at most 168 VGPRs), three blocks per CU -- more
// waves to hide the load and LDS latency, for grids of many blocks.
// FUSED (WPE 2, two register sets, C a multiple of 16, stages of at most
// kFusedStageUnits): the two LDS stages are separate static arrays, so the
// compiler can tell that the stores into one stage do not alias the fragment
// reads of the other, and each channel group's global loads and the previous
// group's LDS stores are interleaved with its MFMAs instead of running as
// phases of their own.
// WD (fused form: 3x3, 64-channel tiles, C % 16 == 0): the weights are read straight from
// the layer's W [O][C][3][3] instead of a channel-grouped copy, so the forward
// needs no relayout launch.  Thread t stages output channel o0 + t/4, channels
// 4 (t%4) .. +3 of the group: 36 contiguous bf16 (9 dword-pair loads), repacked
// per tap into one 8-byte LDS store of 4 channels.
// PC (fused form, 512 threads, WPE 4: two blocks per CU): waves 0-3 only
// multiply (consumers: the accumulators), waves 4-7 only load the next channel
// groups and store them into the other LDS stage (producers, threads 256-511
// serving the load map of threads 0-255); one barrier per group on both sides.
// EPI selects the epilogue at compile time (0 per-element stores, 1 vector
// stores through LDS, 2 lane pairs), so each instance carries the registers of
// one epilogue only.
template <int R, int S, int WM, int XI, int WPE, bool FUSED = false, bool WD = false, bool PC = false, int EPI = 0,
          int FMT = 2>
__global__ __launch_bounds__(PC ? 512 : 256) __attribute__((amdgpu_waves_per_eu(WPE, WPE))) void conv_halo_bf16_kernel(HaloArgs a) {
  using Cfg = HaloCfg<R, S, WM, XI, FMT>;
  static_assert(!PC || FUSED, "producer / consumer split: fused form only");
  static_assert(!WD || (R == 3 && S == 3 && WM == 1 && FMT == 2), "direct weight staging: 3x3, 64-channel tiles");
  static_assert(FMT == 2 || (!FUSED && WM == 1), "32-row tiles: one wave row, not the fused form");
  constexpr int RS = Cfg::RS, BM = Cfg::BM, BN = Cfg::BN, FM = Cfg::FM, FN = Cfg::FN;
  constexpr int SU = FUSED ? kFusedStageUnits : 1;
  // WDMA (fused producer / consumer form on the grouped weight copy): each
  // group's weight tile, one contiguous run of the grouped copy that lands in
  // LDS unchanged, is copied into its stage by LDS DMA (buffer_load ... lds)
  // when the producers store the group's x cells, instead of being loaded into
  // registers two groups ahead and stored by the producers (the two-set
  // producers: at most 2 x items per thread)
  constexpr bool WDMA = PC && FUSED && !WD && XI <= 2;
  __shared__ __attribute__((aligned(16))) u32x4 lds0[SU];
  __shared__ __attribute__((aligned(16))) u32x4 lds1[SU];
  extern __shared__ __attribute__((aligned(16))) u32x4 lds_dyn[];
  u32x4* const lds = FUSED ? lds0 : lds_dyn;

  // wave-uniform (scalar) role: the producer branches and loops stay scalar
  const bool producer = PC && __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) >= 4;
  const int tid = PC ? (int)(threadIdx.x & 255u) : (int)threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar) index
  const int wm = (wave / Cfg::WN) * FM * 32;  // wave's first output channel in the tile
  const int wn = (wave % Cfg::WN) * FN * 32;  // wave's first position in the tile

  // logical block -> (position tile, o tile): the o tiles of one position tile
  // (same x rows) and neighbouring position tiles (shared halo rows) are
  // consecutive, hence on one XCD's L2
  const int lb = xcd_block(a.tiles_m * a.tiles_o);
  const int m0 = (lb / a.tiles_o) * BN;
  const int o0 = (lb % a.tiles_o) * BM;
  const int Wp = a.Wp;
  const int cells = a.xcells;              // x cells per stage (both half-planes)
  const int w_units = BM * Cfg::WPU;       // 16-byte units per weight stage
  const int stage = w_units + cells + 2;   // uint4 per stage; the last 2 units are a
                                           // sink for stores of unused load items
  // stage st: weights at the stage's start, x halo right after them
#define WSM(st) (FUSED ? ((st) ? lds1 : lds0) : lds + (st) * stage)
#define XSM(st) (WSM(st) + w_units)

  // first ext row this block needs: output row of its first position
  uint32_t n_a, pq_a, p_a, q_a;
  a.fPQ.divmod((uint32_t)m0, n_a, pq_a);
  a.fQ.divmod(pq_a, p_a, q_a);
  const int e_start = (int)n_a * a.Hp + (int)p_a;
  const int m_last = min(m0 + BN, a.M) - 1;
  uint32_t n_b, pq_b, p_b, q_b;
  a.fPQ.divmod((uint32_t)m_last, n_b, pq_b);
  a.fQ.divmod(pq_b, p_b, q_b);
  const int rows = (int)n_b * a.Hp + (int)p_b + R - e_start;  // ext rows used by this block

  // first cell of ext row e (block-relative) of half-plane 0: rows of the
  // block's later virtual images sit img_d cells further per image
  auto row_cell = [&](int e) { return e * Wp + ((int)a.fHp.div((uint32_t)(e_start + e)) - (int)n_a) * a.img_d; };

  // whole rows: zero the padding cells once (never written by the loader):
  // per (stage, half-plane, ext row used) the cells [0, pw) and [W + pw, W + 2 pw).
  // Strips load every cell (columns outside the image load as zeros).
  if (a.nstrips == 1) {
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (int i = tid; i < 2 * a.stages * a.rows_max; i += 256) {
      uint32_t sh, e;
      a.fRowsMax.divmod((uint32_t)i, sh, e);
      if ((int)e >= rows) continue;
      u32x4* rowp = XSM(sh >> 1) + (sh & 1) * a.hoff + row_cell((int)e);
      for (int pc = 0; pc < 2 * a.pw; ++pc) rowp[pc < a.pw ? pc : a.W + pc] = z;
    }
  }
  // per-lane cell index of each B fragment column (fixed for the whole block)
  int bcell[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    int m = m0 + wn + j * 32 + (lane & 31);
    int cidx = 0;
    if (m < a.M) {
      uint32_t n, pq, p, q;
      a.fPQ.divmod((uint32_t)m, n, pq);
      a.fQ.divmod(pq, p, q);
      cidx = ((int)n * a.Hp + (int)p - e_start) * Wp + ((int)n - (int)n_a) * a.img_d + (int)q + a.cs;
    }
    bcell[j] = cidx;
  }

  const int HW = a.H * a.W;

  // x load items (fixed for the whole block; only the channel group moves):
  // item -> (half, ext row e, column pair wi).  The first XITER/2 items of a
  // thread are in the lower half-plane (channels 0-7 of the group), the others
  // in the upper one, so a channel's validity is uniform per load.  x_voff is
  // the byte offset of the item's first element at channel 0 (+8 channels for
  // the upper half), or an offset past the end of the buffer for rows outside
  // the image.
  const int HW2 = HW * 2;  // bytes per channel plane
  const __amdgpu_buffer_rsrc_t xrsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.x_bytes, 0x00020000);
  // zero-length buffer: every load through it returns 0 (masked channels and groups)
  const __amdgpu_buffer_rsrc_t zrsrc = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, 0, 0x00020000);
  constexpr int XH = Cfg::XITER / 2;  // items per thread per half-plane
  int x_voff[Cfg::XITER], x_loff[Cfg::XITER];
#pragma unroll
  for (int it = 0; it < Cfg::XITER; ++it) {
    const int half = it < XH ? 0 : 1;
    const uint32_t i = (uint32_t)(tid + (it - half * XH) * 256);
    uint32_t wi, e;
    a.fW2.divmod(i, e, wi);
    int voff = (int)0x80000000u, loff = -1;
    if ((int)e < rows) {
      uint32_t eg = (uint32_t)(e_start + (int)e), vimg, hr, n, strip;
      a.fHp.divmod(eg, vimg, hr);
      a.fStrips.divmod(vimg, n, strip);
      const int h = (int)hr - a.ph;
      // input columns of the pair (even, W even: both inside or both outside)
      const int col = (int)strip * a.TW + a.lcol0 + 2 * (int)wi;
      if (h >= 0 && h < a.H && col >= 0 && col < a.W)
        voff = (int)((((long)n * a.C + half * 8) * HW + (long)h * a.W + col) * 2);
      loff = half * a.hoff + (int)e * Wp + ((int)vimg - (int)n_a) * a.img_d + a.lcell0 + 2 * (int)wi;
    }
    x_voff[it] = voff;
    x_loff[it] = loff >= 0 ? loff : cells;  // unused items store to the sink
  }

  const bool full_o = o0 + BM <= a.O;  // uniform: no per-row checks needed
  // W load items, fixed for the block: byte offset of the 16-byte unit in
  // channel group 0 (out of range for rows past O) and its LDS unit index.  The
  // grouped copy has the LDS tile's pitch, so unit u of the tile is unit u of
  // the LDS stage: consecutive lanes load and store consecutive units.
  const int OGP = a.O * Cfg::WPU;  // bytes per channel of the grouped weights: group offset = c0 * OGP
  const __amdgpu_buffer_rsrc_t wrsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.wt, (short)0, a.w_bytes, 0x00020000);
  int w_goff[Cfg::WITER], w_loff[Cfg::WITER];
  // WD: byte offset of the thread's 36 weights at channel group 0 (group
  // offset c0 * 18), and the LDS byte offset of its tap-0 store
  int wd_goff = 0, wd_loff = 0;
  if constexpr (WD) {
    // wave w stages rows 16w .. 16w+15, lanes 0-31 the even ones and lanes
    // 32-63 the odd ones: rows 19 units apart, 8 even rows cover all 64 banks
    // once per 8-byte store, where 8 consecutive rows overlap (measured: two
    // cycles per ds_write_b64 instead of one)
    const int o = (tid >> 6) * 16 + 2 * ((tid >> 2) & 7) + ((tid >> 5) & 1), q = tid & 3;
    wd_goff = o0 + o < a.O ? ((o0 + o) * a.C + 4 * q) * 18 : (int)0x80000000u;
    wd_loff = (o * Cfg::WPU + (q >> 1)) * 16 + (q & 1) * 8;
  }
#pragma unroll
  for (int it = 0; it < (WD ? 0 : Cfg::WITER); ++it) {
    const int u = tid + it * 256;
    const bool ok = u < Cfg::WUNITS && (full_o || o0 + u / Cfg::WPU < a.O);
    w_goff[it] = ok ? (o0 * Cfg::WPU + u) * 16 : (int)0x80000000u;
    w_loff[it] = u < Cfg::WUNITS ? u : w_units + cells;  // sink
  }

  // With two register sets (DEPTH 2) the global loads of channel group kt+2
  // are issued while group kt is multiplied and group kt+1 is written to LDS,
  // so every load has two compute phases to arrive; wide tiles (more than 4 x or 5 weight load
  // items per thread) keep one set to stay within two waves' registers.
  // (PC: the producers keep two sets for narrow loads -- the loads of group k are
  // issued two multiply phases before the group is stored -- and both roles fit
  // 128 registers; with 4 x items per thread one set, which fits without spills)
  constexpr int DEPTH = PC ? (Cfg::XITER <= 2 ? 2 : 1) : (WPE == 2 && Cfg::XITER <= 4 && Cfg::WITER <= 5) ? 2 : 1;
  static_assert(!FUSED || PC || DEPTH == 2, "the fused form keeps two register sets");
  u32x4 wreg[DEPTH][WD ? 1 : Cfg::WITER];
  u32x2 wdr[DEPTH][WD ? 9 : 1];
  uint32_t xreg[DEPTH][Cfg::XITER][8];
  // Loads of channel group c0 .. c0+15.  Every load is issued (no branches, so
  // the compiler's wait counts stay exact across the pipeline): channels past C
  // and groups past the last one read through the zero-length buffer.
  auto gload = [&](auto SET, int c0_) {
    constexpr int sI = decltype(SET)::value;
    // the group's channel offset goes into the scalar offset operand: keep it in
    // a scalar register (a per-lane value there costs a loop per load)
    const int c0 = __builtin_amdgcn_readfirstlane(c0_);
    const int crem = a.C - c0;  // channels left from c0 (<= 0 past the last group)
    // groups past the last one (c0 >= C) read zeros through the zero-length
    // buffer: the channel offset is a scalar offset, which is not range-checked
    if constexpr (WD) {
#pragma unroll
      for (int j = 0; j < 9; ++j)
        wdr[sI][j] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                                   crem > 0 ? wrsrc : zrsrc, wd_goff + 8 * j, c0 * 18, 0));
    } else if constexpr (!WDMA) {
#pragma unroll
      for (int it = 0; it < Cfg::WITER; ++it)
        wreg[sI][it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                     crem > 0 ? wrsrc : zrsrc, w_goff[it], c0 * OGP, 0));
    }
#pragma unroll
    for (int it = 0; it < Cfg::XITER; ++it) {
      const int half = it < XH ? 0 : 1;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        xreg[sI][it][j] = __builtin_amdgcn_raw_buffer_load_b32(j + 8 * half < crem ? xrsrc : zrsrc,
                                                               x_voff[it], (c0 + j) * HW2, 0);
    }
  };
  auto sstore = [&](auto SET, int st) {
    constexpr int sI = decltype(SET)::value;
    // unconditional stores (masked items go to the sink), so the wait for the
    // older register set does not also wait for the loads issued after it
    if constexpr (WD) {
      // dword k of the 18 loaded holds elements 2k, 2k+1 (element e = channel
      // e / 9, tap e % 9); tap t takes elements t, 9+t, 18+t, 27+t
      auto dw = [&](int k) { return wdr[sI][k >> 1][k & 1]; };
      auto two = [&](int e0, int e1) {  // bf16 e0 low, e1 high
        const uint32_t sel = (2u * (e0 & 1)) | ((2u * (e0 & 1) + 1u) << 8) | ((4u + 2u * (e1 & 1)) << 16) |
                             ((5u + 2u * (e1 & 1)) << 24);
        return __builtin_amdgcn_perm(dw(e1 >> 1), dw(e0 >> 1), sel);
      };
      char* wb = reinterpret_cast<char*>(WSM(st)) + wd_loff;
#pragma unroll
      for (int t = 0; t < 9; ++t) {
        u32x2 v;
        v[0] = two(t, 9 + t);
        v[1] = two(18 + t, 27 + t);
        *reinterpret_cast<u32x2*>(wb + t * 32) = v;
      }
    } else if constexpr (!WDMA) {
#pragma unroll
      for (int it = 0; it < Cfg::WITER; ++it) WSM(st)[w_loff[it]] = wreg[sI][it];
    }
    // Each item is two adjacent cells (a column pair).  Consecutive lanes hold
    // consecutive pairs, so storing every lane's first cell together would hit
    // every other 16-byte cell (two-way bank conflicts); lanes whose bit 2
    // differs from bit 3 store their second cell first, which makes each group
    // of 8 (and of 16) lanes cover distinct banks.
    const bool xsw = ((lane >> 2) ^ (lane >> 3)) & 1;
#pragma unroll
    for (int it = 0; it < Cfg::XITER; ++it) {
      {
        const uint32_t* xr = xreg[sI][it];
        u32x4 c0v, c1v;
        c0v.x = pack_lo(xr[0], xr[1]); c0v.y = pack_lo(xr[2], xr[3]);
        c0v.z = pack_lo(xr[4], xr[5]); c0v.w = pack_lo(xr[6], xr[7]);
        c1v.x = pack_hi(xr[0], xr[1]); c1v.y = pack_hi(xr[2], xr[3]);
        c1v.z = pack_hi(xr[4], xr[5]); c1v.w = pack_hi(xr[6], xr[7]);
        u32x4* base = XSM(st) + x_loff[it];
        base[xsw ? 1 : 0] = xsw ? c1v : c0v;
        base[xsw ? 0 : 1] = xsw ? c0v : c1v;
      }
    }
  };

  // WDMA: copy group g's weight tile (units 0 .. WUNITS-1 of the stage; rows
  // past O read zeros) into stage st; copy instruction c = wave + 4 i covers
  // units 64c .. 64c+63
  auto wdma = [&](int st, int g) {
    if constexpr (WDMA) {
      const uint32_t la = lds_byte_addr(WSM(st));
      const int soff = __builtin_amdgcn_readfirstlane(16 * g * OGP);
#pragma unroll
      for (int c = wave; c < (Cfg::WUNITS + 63) / 64; c += 4) {
        const int u = 64 * c + lane;
        const bool ok = u < Cfg::WUNITS && (full_o || o0 + u / Cfg::WPU < a.O);
        if (u < Cfg::WUNITS) lds_copy16(wrsrc, ok ? (o0 * Cfg::WPU + u) * 16 : (int)0x80000000u, soff, la + c * 1024);
      }
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int half_l = lane >> 5, row_l = lane & 31;
  auto compute = [&](int st) {
    const u32x4* Wp_ = WSM(st) + (wm + row_l) * Cfg::WPU + half_l;
    const u32x4* Xp_ = XSM(st) + half_l * a.hoff;
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int tap = r * S + s;
        const int toff = r * Wp + s;
        bf16x8 af[FM], bfr[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i) af[i] = __builtin_bit_cast(bf16x8, Wp_[i * 32 * Cfg::WPU + tap * 2]);
#pragma unroll
        for (int j = 0; j < FN; ++j) bfr[j] = __builtin_bit_cast(bf16x8, Xp_[bcell[j] + toff]);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
      }
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;

  // Channel groups kt = 0 .. nk-1, LDS buffer kt & 1.  DEPTH 2 invariant at an
  // even kt: buffer 0 holds group kt, register set 1 holds group kt+1 (in
  // flight), set 0 is free.  The steady-state loop issues its loads without
  // conditions so that each wait covers only the older register set.
  const int nk = (a.C + 15) / 16;
  if constexpr (PC) {
    // group kt is multiplied from stage kt & 1 while the producers store group
    // kt+1 into the other stage (read by the consumers before the previous
    // barrier) and load group kt+2 (fused form: every group is whole, C % 16 == 0)
    if (producer && DEPTH == 1) {
      gload(I0{}, 0);
      __builtin_amdgcn_sched_barrier(0);
      sstore(I0{}, 0);
      if (nk > 1) gload(I0{}, 16);
      __syncthreads();
      for (int kt = 0; kt < nk; kt += 2) {
        if (kt + 1 < nk) sstore(I0{}, 1);
        if (kt + 2 < nk) gload(I0{}, (kt + 2) * 16);
        __syncthreads();
        if (kt + 1 >= nk) break;
        if (kt + 2 < nk) sstore(I0{}, 0);
        if (kt + 3 < nk) gload(I0{}, (kt + 3) * 16);
        __syncthreads();
      }
      return;
    }
    if constexpr (DEPTH == 2) if (producer) {
      // two register sets: at an even kt set 1 holds group kt+1 and set 0
      // group kt+2 (in flight).  Every load is issued (groups past the last
      // read zeros), so each wait covers only the set about to be stored.
      // swap: the LDS stores of one register set with the loads of its next
      // group into the same registers, alternating item by item, so that the
      // address unit works on this wave's loads while its stores go to LDS.
      auto swap = [&](auto SET, int st, int c0n) {
        sstore(SET, st);
        wdma(st, c0n / 16 - 2);  // the group just stored
        gload(SET, c0n);
        // WDMA: the copy is older than this set's x loads, which may stay in flight
        if constexpr (WDMA) wait_vmcnt<Cfg::XITER * 8>();
        constexpr int NW = WD ? 9 : WDMA ? 0 : Cfg::WITER;
#pragma unroll
        for (int i = 0; i < NW; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS store
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
        }
#pragma unroll
        for (int it = 0; it < Cfg::XITER; ++it) {
          __builtin_amdgcn_sched_group_barrier(0x200, 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, 8, 0);
        }
      };
      gload(I0{}, 0);
      gload(I1{}, 16);
      __builtin_amdgcn_sched_barrier(0);
      swap(I0{}, 0, 32);
      __syncthreads();
      int kt = 0;
      for (; kt + 2 < nk; kt += 2) {
        swap(I1{}, 1, (kt + 3) * 16);
        __syncthreads();
        swap(I0{}, 0, (kt + 4) * 16);
        __syncthreads();
      }
      // nk - kt (1 or 2) barriers left: one per remaining group of the consumers
      if (kt + 1 < nk) {
        sstore(I1{}, 1);
        wdma(1, kt + 1);
        if constexpr (WDMA) wait_vmcnt<0>();
        __syncthreads();
      }
      __syncthreads();
      return;
    }
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      // fragment reads of tap t+LA placed between the MFMAs of tap t, so each
      // read has LA taps of MFMAs to arrive (LA = VH_HALO_PC_LA)
      compute(kt & 1);
      constexpr int LA = VH_HALO_PC_LA;
      if constexpr (LA > 0) {
        __builtin_amdgcn_sched_group_barrier(0x100, LA * (FM + FN), 0);  // reads of taps 0 .. LA-1
#pragma unroll
        for (int t = 0; t < RS; ++t) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (t + LA < RS) __builtin_amdgcn_sched_group_barrier(0x100, (FM + FN) / 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (t + LA < RS) __builtin_amdgcn_sched_group_barrier(0x100, (FM + FN) / 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, FM * FN - 2, 0);
        }
      }
      __syncthreads();
    }
  } else if constexpr (DEPTH == 2) {
    gload(I0{}, 0);
    gload(I1{}, FUSED && nk < 2 ? 0 : 16);  // all zeros when there is a single group
    __builtin_amdgcn_sched_barrier(0);
    sstore(I0{}, 0);
    __syncthreads();
    int kt = 0;
    // Fused form: one channel group = the MFMAs of stage ST, with the loads of
    // group +2 and the LDS stores of group +1 (into the other stage) placed
    // between them: per tap, 4 MFMAs with 3 global loads, one LDS store and
    // the fragment reads of the tap after next in the gaps.
    // LDS stores per group (WD: 9 weight stores + 2 per x item, spread over the taps)
    constexpr int NDSW = WD ? 9 + 2 * Cfg::XITER : 0;
    auto fused = [&](auto ST, auto LSET, int lc0, auto SSET) {
      constexpr int st = decltype(ST)::value;
      gload(LSET, lc0);
      sstore(SSET, 1 - st);
      compute(st);
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * (FM + FN), 0);  // fragment reads of taps 0, 1
#pragma unroll
      for (int t = 0; t < RS; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);  // global loads
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (t + 2 < RS) __builtin_amdgcn_sched_group_barrier(0x100, (FM + FN) / 2, 0);  // LDS reads
        // LDS stores: one per tap (WD: NDSW spread over the taps)
        if (WD && t < NDSW % RS) __builtin_amdgcn_sched_group_barrier(0x200, WD ? NDSW / RS + 1 : 1, 0);
        else __builtin_amdgcn_sched_group_barrier(0x200, WD ? NDSW / RS : 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        if (t + 2 < RS) __builtin_amdgcn_sched_group_barrier(0x100, (FM + FN) / 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
    };
    if constexpr (FUSED) {
      for (; kt + 3 < nk; kt += 2) {
        fused(I0{}, I0{}, (kt + 2) * 16, I1{});
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        fused(I1{}, I1{}, (kt + 3) * 16, I0{});
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
      }
    }
    // sched_barrier(0) keeps the compiler from sinking the loads to their
    // use (which would leave them no time to arrive)
    for (; !FUSED && kt + 3 < nk; kt += 2) {
      gload(I0{}, (kt + 2) * 16);
      __builtin_amdgcn_sched_barrier(0);
      compute(0);
      __builtin_amdgcn_sched_barrier(0);
      sstore(I1{}, 1);
      __syncthreads();
      gload(I1{}, (kt + 3) * 16);
      __builtin_amdgcn_sched_barrier(0);
      compute(1);
      __builtin_amdgcn_sched_barrier(0);
      sstore(I0{}, 0);
      __syncthreads();
    }
    const int rem = nk - kt;  // 1, 2 or 3 groups left
    if (!FUSED || rem == 3) gload(I0{}, (kt + 2) * 16);  // zeros unless rem == 3
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
  } else if (WPE == 3) {
    // one LDS stage: the next group's loads are in flight during the compute;
    // a barrier before its store (every wave done reading) and one after it
    gload(I0{}, 0);
    sstore(I0{}, 0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      if (kt + 1 < nk) gload(I0{}, (kt + 1) * 16);
      __builtin_amdgcn_sched_barrier(0);
      compute(0);
      __builtin_amdgcn_sched_barrier(0);
      if (kt + 1 < nk) {
        __syncthreads();
        sstore(I0{}, 0);
        __syncthreads();
      }
    }
  } else {
    gload(I0{}, 0);
    sstore(I0{}, 0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      if (kt + 1 < nk) gload(I0{}, (kt + 1) * 16);
      __builtin_amdgcn_sched_barrier(0);
      compute(kt & 1);
      __builtin_amdgcn_sched_barrier(0);
      if (kt + 1 < nk) sstore(I0{}, (kt + 1) & 1);
      __syncthreads();
    }
  }

#undef WSM
#undef XSM
  const int PQ = a.P * a.Q;
  // fp32 bias of the 16 accumulator rows of fragment row i of this lane (output
  // channel o0 + wm + i*32 + (v>>2)*8 + (lane>>5)*4 + (v&3)), loaded per i: one
  // uniform branch, buffer loads that return 0 past O (the whole offset in the
  // per-lane operand: the scalar offset is not range-checked).
  const __amdgpu_buffer_rsrc_t brsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.bias, (short)0, a.bias ? a.O * 2 : 0, 0x00020000);
  auto load_bias = [&](int i, float (&bi)[16]) {
#pragma unroll
    for (int v = 0; v < 16; ++v) bi[v] = 0.f;
    if (a.bias) {
      const int ob = (o0 + wm + i * 32 + (lane >> 5) * 4) * 2;
#pragma unroll
      for (int v = 0; v < 16; ++v)
        bi[v] = bf16_to_f32((uint16_t)__builtin_amdgcn_raw_buffer_load_b16(brsrc, ob + ((v >> 2) * 8 + (v & 3)) * 2, 0, 0));
    }
  };
  if constexpr (EPI == 2) {
    // Pair epilogue.  Accumulator v of a lane is output row (v>>2)*8 + (v&3)
    // (+4 in the upper half-wave) at the lane's position.  Lanes 2m and 2m+1
    // hold consecutive positions (the same image row: Q and every tile start
    // are even); they swap one value of the rows v and v+1 (v even) so that the
    // even lane holds row v and the odd lane row v+1, each at both positions,
    // and store them as one dword: 32 dword stores per lane, no LDS.  fp32
    // bias add and activation before the single rounding to bf16.
    const int PQ2 = PQ * 2;
    const bool odd = lane & 1;
    const __amdgpu_buffer_rsrc_t yrsrc = __builtin_amdgcn_make_buffer_rsrc((void*)a.y, (short)0, a.y_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t mrsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)(a.act == 2 ? a.mask : a.y), (short)0, a.y_bytes, 0x00020000);
    int yoff[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      // the pair's first (even) position
      uint32_t m = (uint32_t)(m0 + wn + j * 32 + (lane & 30)), vimg, pq, p, ql, n, strip;
      a.fPQ.divmod(m, vimg, pq);
      a.fQ.divmod(pq, p, ql);
      a.fStrips.divmod(vimg, n, strip);
      const int q = (int)strip * a.TW + (int)ql;
      yoff[j] = (int)m < a.M && q < a.Q
                    ? (int)((n * (uint32_t)a.O * (uint32_t)PQ + p * (uint32_t)a.Q + (uint32_t)q) * 2u) +
                          ((lane >> 5) * 4 + (lane & 1)) * PQ2
                    : (int)0x80000000u;
    }
    // the ReLU-backward mask of the dwords this lane stores, all loaded before the first store
    uint32_t mk[FM][FN][8];
    if (a.act == 2) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int vp = 0; vp < 8; ++vp) {
          const int orow = o0 + wm + i * 32 + (vp >> 1) * 8 + (vp & 1) * 2;
#pragma unroll
          // the row offset goes into the range-checked per-lane offset: rows past O
          // (last o tile) and positions past the end read zeros
          for (int j = 0; j < FN; ++j)
            mk[i][j][vp] = __builtin_amdgcn_raw_buffer_load_b32(mrsrc, (int)((uint32_t)yoff[j] + (uint32_t)(orow * PQ2)), 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      float bv[16];
      load_bias(i, bv);
#pragma unroll
      for (int vp = 0; vp < 8; ++vp) {
        const int v = 2 * vp;  // rows v, v+1 = orow, orow+1
        const int orow = o0 + wm + i * 32 + (v >> 2) * 8 + (v & 3);  // wave-uniform part of o
        const bool ok = full_o || orow + (lane >> 5) * 4 + (lane & 1) < a.O;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          float a0 = acc[i][j][v] + bv[v], a1 = acc[i][j][v + 1] + bv[v + 1];
          if (a.act == 1) {
            a0 = fmaxf(a0, 0.f);
            a1 = fmaxf(a1, 0.f);
          }
          // the even lane needs its partner's row-v value, the odd lane its partner's row-(v+1) value
          const float recv = __builtin_bit_cast(
              float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, odd ? a0 : a1), 0xB1, 0xF, 0xF, false));
          const float lo = odd ? recv : a0, hi = odd ? a1 : recv;
          uint32_t d = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)lo) |
                       ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)hi) << 16);
          if (a.act == 2) {
            const uint32_t m = mk[i][j][vp];
            d &= (bf16_to_f32((uint16_t)(m & 0xffffu)) > 0.f ? 0x0000ffffu : 0u) |
                 (bf16_to_f32((uint16_t)(m >> 16)) > 0.f ? 0xffff0000u : 0u);
          }
          if (ok) __builtin_amdgcn_raw_buffer_store_b32(d, yrsrc, yoff[j], orow * PQ2, 0);
        }
      }
    }
    return;
  }
  if constexpr (EPI == 1) {
    // Vector epilogue.  Each wave writes its FM*32 o x 64 position tile, bias added
    // and rounded once to bf16 (ReLU applied in fp32 first), into its own LDS
    // region [o][position] (pitch 72 elements: the two half-waves, 4 rows
    // apart, fall on disjoint banks), then stores runs of 8 consecutive
    // positions (16 bytes) per lane.  P*Q % 8 == 0, so a run never crosses an
    // image and its address is 16-byte aligned.
    constexpr int EP = 72;
    if constexpr (!PC) __syncthreads();  // every wave has finished reading the last stage
                                         // (PC: the consumers' last loop barrier)
    uint16_t* eb = reinterpret_cast<uint16_t*>(lds) + wave * (64 * EP);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      float bv[16];
      load_bias(i, bv);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = i * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          float val = acc[i][j][v] + bv[v];
          if (a.act == 1) val = fmaxf(val, 0.f);
          eb[row * EP + j * 32 + (lane & 31)] = __builtin_bit_cast(uint16_t, (__bf16)val);
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
    // lane -> 8 positions m .. m+7 (the same for every pass) and rows it*8 + lane/8:
    // all eight LDS reads first, then the stores
    const int k8 = lane & 7, m = m0 + wn + k8 * 8;
    uint32_t n_e, pq_e;
    a.fPQ.divmod((uint32_t)min(m, a.M - 1), n_e, pq_e);
    const long ybase = (long)n_e * a.O * PQ + pq_e;
    uint4 ev[FM * 4];
#pragma unroll
    for (int it = 0; it < FM * 4; ++it)
      ev[it] = *reinterpret_cast<const uint4*>(eb + (it * 8 + (lane >> 3)) * EP + k8 * 8);
#pragma unroll
    for (int it = 0; it < FM * 4; ++it) {
      const int row = it * 8 + (lane >> 3);
      const int o = o0 + wm + row;
      if (o < a.O && m < a.M) {
        const long off = ybase + (long)o * PQ;
        uint4 val = ev[it];
        if (a.act == 2) {
          // zero where the layer's forward output (the mask) is not positive
          const uint4 mk = *reinterpret_cast<const uint4*>(a.mask + off);
          uint32_t* vv = reinterpret_cast<uint32_t*>(&val);
          const uint32_t* mm = reinterpret_cast<const uint32_t*>(&mk);
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const uint32_t lo = bf16_to_f32((uint16_t)(mm[d] & 0xffffu)) > 0.f ? 0x0000ffffu : 0u;
            const uint32_t hi = bf16_to_f32((uint16_t)(mm[d] >> 16)) > 0.f ? 0xffff0000u : 0u;
            vv[d] &= lo | hi;
          }
        }
        *reinterpret_cast<uint4*>(a.y + off) = val;
      }
    }
    return;
  }
  // epilogue: rows = o (acc_row), cols = positions (lane & 31); fp32 bias add,
  // one rounding to bf16, NCHW store (lanes walk consecutive q).  Buffer stores:
  // the per-lane offset is the position (plus 4 rows for the upper half-wave),
  // the output-channel row is a scalar offset; positions past the end carry an
  // out-of-range offset and their stores are dropped.
  const int PQ2 = PQ * 2;
  const __amdgpu_buffer_rsrc_t yrsrc = __builtin_amdgcn_make_buffer_rsrc((void*)a.y, (short)0, a.y_bytes, 0x00020000);
  int yoff[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    uint32_t m = (uint32_t)(m0 + wn + j * 32 + (lane & 31)), vimg, pq, p, ql, n, strip;
    a.fPQ.divmod(m, vimg, pq);
    a.fQ.divmod(pq, p, ql);
    a.fStrips.divmod(vimg, n, strip);
    const int q = (int)strip * a.TW + (int)ql;
    yoff[j] = (int)m < a.M && q < a.Q
                  ? (int)((n * (uint32_t)a.O * (uint32_t)PQ + p * (uint32_t)a.Q + (uint32_t)q) * 2u) +
                        (lane >> 5) * 4 * PQ2
                  : (int)0x80000000u;
  }
  const __amdgpu_buffer_rsrc_t mrsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)(a.act == 2 ? a.mask : a.y), (short)0, a.y_bytes, 0x00020000);
  // fp32 result + bias, then the fused activation: ReLU (NaN -> 0, as fmaxf),
  // or the ReLU backward of the layer below (zero where its output, the mask,
  // is not positive).  The mask values are all loaded before the first store
  // (a load may not pass a store to possibly the same memory).
  uint32_t keep[FM][FN] = {};  // bit v: mask value of accumulator v is positive
  if (a.act == 2) {
    uint16_t mv[FM][FN][16];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int orow = o0 + wm + i * 32 + (v >> 2) * 8 + (v & 3);
#pragma unroll
        for (int j = 0; j < FN; ++j)  // row offset range-checked too (rows past O read zeros)
          mv[i][j][v] = __builtin_amdgcn_raw_buffer_load_b16(mrsrc, (int)((uint32_t)yoff[j] + (uint32_t)(orow * PQ2)), 0, 0);
      }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) keep[i][j] |= (bf16_to_f32(mv[i][j][v]) > 0.f ? 1u : 0u) << v;
  }
  auto epi = [&](float val, int i, int j, int v) {
    if (a.act == 1) val = fmaxf(val, 0.f);
    else if (a.act == 2 && !((keep[i][j] >> v) & 1u)) val = 0.f;
    return __builtin_bit_cast(uint16_t, (__bf16)val);
  };
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    float bv[16];
    load_bias(i, bv);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int orow = o0 + wm + i * 32 + (v >> 2) * 8 + (v & 3);  // wave-uniform part of o
      const bool ok = full_o || orow + (lane >> 5) * 4 < a.O;
#pragma unroll
      for (int j = 0; j < FN; ++j)
        if (ok)
          __builtin_amdgcn_raw_buffer_store_b16(epi(acc[i][j][v] + bv[v], i, j, v), yrsrc, yoff[j], orow * PQ2, 0);
    }
  }
}


// ---------------------------------------------------------------- host side
namespace {

template <int R, int S, int WM, int XI, int WPE = 2, bool FUSED = false, bool WD = false, bool PC = false,
          int FMT = 2>
int launch_halo(const HaloArgs& a, size_t lds_bytes, hipStream_t st) {
  using Cfg = HaloCfg<R, S, WM, XI, FMT>;
  auto k0 = conv_halo_bf16_kernel<R, S, WM, XI, WPE, FUSED, WD, PC, 0, FMT>;
  auto k1 = conv_halo_bf16_kernel<R, S, WM, XI, WPE, FUSED, WD, PC, 1, FMT>;
  auto k2 = conv_halo_bf16_kernel<R, S, WM, XI, WPE, FUSED, WD, PC, 2, FMT>;
  // the fused form's stages are static (2 x 38.9 KB): no dynamic LDS
  if (!FUSED) {
    VH_LDS_LIMIT_ONCE(k0);
    VH_LDS_LIMIT_ONCE(k1);
    VH_LDS_LIMIT_ONCE(k2);
  }
  auto kern = a.vec_epi ? k1 : a.pair_epi ? k2 : k0;
  HaloArgs g = a;
  g.tiles_m = (a.M + Cfg::BN - 1) / Cfg::BN;
  g.tiles_o = (a.O + Cfg::BM - 1) / Cfg::BM;
  kern<<<dim3((unsigned)(g.tiles_m * g.tiles_o)), PC ? 512 : 256, FUSED ? 0 : lds_bytes, st>>>(g);
  VH_LAUNCH_CHECK();
  return VH_OK;
}

// x load items per thread: an even count, half of them per half-plane
int halo_xi(const HaloArgs& a) { return 2 * ((a.rows_max * a.npairs + 255) / 256); }

template <int R, int S, int WM, int FMT = 2>
int pick_xi(const HaloArgs& a, size_t lds_bytes, hipStream_t st) {
  const int xi = halo_xi(a);
  if (xi <= 2) return launch_halo<R, S, WM, 2, 2, false, false, false, FMT>(a, lds_bytes, st);
  if (xi <= 4) return launch_halo<R, S, WM, 4, 2, false, false, false, FMT>(a, lds_bytes, st);
  if (xi <= 6) return launch_halo<R, S, WM, 6, 2, false, false, false, FMT>(a, lds_bytes, st);
  return launch_halo<R, S, WM, 8, 2, false, false, false, FMT>(a, lds_bytes, st);
}

// three blocks per CU: the 3x3 load widths that fit 168 VGPRs without spills
int pick_xi_wpe3(const HaloArgs& a, int WM, int FM, size_t lds_bytes, hipStream_t st) {
  const int xi = halo_xi(a);
  if (FM == 1)
    return xi <= 2 ? launch_halo<3, 3, 1, 2, 3, false, false, false, 1>(a, lds_bytes, st)
                   : launch_halo<3, 3, 1, 4, 3, false, false, false, 1>(a, lds_bytes, st);
  if (WM == 2) return launch_halo<3, 3, 2, 2, 3>(a, lds_bytes, st);
  return xi <= 2 ? launch_halo<3, 3, 1, 2, 3>(a, lds_bytes, st) : launch_halo<3, 3, 1, 4, 3>(a, lds_bytes, st);
}

}  // namespace

// Exact maximum number of ext rows any block of BN positions spans (positions
// of P x TW virtual images, Hp ext rows per image, R taps).  The scan over all
// blocks costs tens of microseconds of host time at the configs' sizes, so the
// results are kept per shape (a small table, replaced round-robin).
int halo_rows_max(long Mv, int BN, long PQv, int TW, int Hp, int R) {
  struct Entry {
    long Mv, PQv;
    int BN, TW, Hp, R, rows_max;
  };
  static std::mutex mu;
  static Entry table[64];
  static int used = 0, next = 0;
  {
    std::lock_guard<std::mutex> lk(mu);
    for (int i = 0; i < used; ++i) {
      const Entry& e = table[i];
      if (e.Mv == Mv && e.PQv == PQv && e.BN == BN && e.TW == TW && e.Hp == Hp && e.R == R) return e.rows_max;
    }
  }
  int rows_max = 0;
  for (long m0 = 0; m0 < Mv; m0 += BN) {
    const long ml = std::min(m0 + BN, Mv) - 1;
    const long ra = (m0 / PQv) * Hp + (m0 % PQv) / TW, rb = (ml / PQv) * Hp + (ml % PQv) / TW;
    rows_max = std::max(rows_max, (int)(rb + R - ra));
  }
  std::lock_guard<std::mutex> lk(mu);
  table[next] = Entry{Mv, PQv, BN, TW, Hp, R, rows_max};
  next = (next + 1) % 64;
  if (used < 64) ++used;
  return rows_max;
}

// Returns VH_ERR_UNSUPPORTED (without launching) when the shape is outside what
// the halo kernel handles; the caller then uses the generic implicit GEMM.
size_t halo_conv_bf16_ws(int C, int O, int R, int S) { return (size_t)((C + 15) / 16) * O * (2 * R * S + 1) * 16; }

int halo_conv_bf16(const void* x, const void* w, int w_mode, void* ws, const void* bias, void* y, int N, int C,
                   int H, int W, int O, int R, int S, int ph, int pw, hipStream_t st, int act, const void* mask) {
  const int P = H + 2 * ph - R + 1, Q = W + 2 * pw - S + 1;
  if (P <= 0 || Q <= 0) return VH_ERR_UNSUPPORTED;
  if (C < 1 || (W % 2) != 0 || ph > R - 1 || pw > S - 1) return VH_ERR_UNSUPPORTED;
  const int nk = (C + 15) / 16;  // channel groups; the grouped weights are padded with zeros to whole groups
  if (!((R == 3 && S == 3) || (R == 5 && S == 5) || (R == 1 && S == 1))) return VH_ERR_UNSUPPORTED;
  // 3x3 with at most 64 input and 33-64 output channels: the resident-weight
  // kernel (vh_wres.hip) for the masked input gradient (act 2), where it
  // measured faster; VOLTA_HIP_WRES=1 sends every shape in its envelope there, 0 none.
  if (R == 3 && S == 3 && C <= 64 && O <= 64) {
    const char* e = getenv("VOLTA_HIP_WRES");
    const int mode = e && *e ? (*e == '0' ? 0 : 1) : -1;
    // (at most 32 output channels: the 32-row halo tiles measured faster, 68.2 -> 49.6 us for
    // configs[4]'s 32 -> 27 input gradient)
    if (mode == 1 || (mode == -1 && act == 2 && O > 32)) {
      const int r = wres_conv_bf16(x, w, w_mode, ws, bias, y, N, C, H, W, O, ph, pw, st, act, mask);
      if (r != VH_ERR_UNSUPPORTED) return r;
    }
  }
  const void* wt = ws;
  HaloArgs a;
  a.x = (const uint16_t*)x;
  a.wt = (const uint16_t*)wt;
  a.bias = (const uint16_t*)bias;
  a.y = (uint16_t*)y;
  a.act = act;
  a.mask = (const uint16_t*)mask;
  a.N = N; a.C = C; a.H = H; a.W = W; a.O = O; a.P = P; a.Q = Q; a.ph = ph; a.pw = pw;
  a.Hp = H + 2 * ph;  // = P + R - 1
  const long xb = (long)N * C * H * W * 2;
  if (xb >= (1L << 31) - 16) return VH_ERR_UNSUPPORTED;  // 32-bit buffer offsets
  a.x_bytes = (int)xb;
  const long yb_ = (long)N * O * P * Q * 2;
  if (yb_ >= (1L << 31) - 16) return VH_ERR_UNSUPPORTED;
  a.y_bytes = (int)yb_;
  const long wb = (long)nk * O * (2 * R * S + 1) * 16;
  if (wb >= (1L << 31) - 16) return VH_ERR_UNSUPPORTED;
  a.w_bytes = (int)wb;
  a.fHp = FastDiv((uint32_t)a.Hp);
  a.stages = nk == 1 ? 1 : 2;  // a single channel group needs no second buffer

  // Tile shape: 64 output channels x 256 positions (WM 1) or 128 x 128 (WM 2),
  // over whole rows or over column strips of TW columns.  Preference: two
  // blocks per CU (LDS <= 80 KB), then the fewest computed columns (strips
  // past Q are waste), then the fewest staged input cells per block.
  struct Cand {
    int TW, WM, rows_max, Wr, Wp, img_d, xcells;  // Wr: cells per row and half-plane
    size_t lds;
    long cols;  // virtual columns per row: nstrips * TW
  };
  // 3x3 layers with at most 32 output channels take 32-row tiles (one wave row
  // of 32 x 64 wave tiles): a 64-row tile would leave half its MFMA work empty
  const int fm = R == 3 && S == 3 && O <= 32 ? 1 : 2;
  auto eval = [&](int TW, int WM, Cand& c) {
    const int BN = (4 / WM) * 64, BM = WM * fm * 32;
    const int nstrips = (Q + TW - 1) / TW;
    const long Mv = (long)N * nstrips * P * TW;
    if (Mv >= (1L << 31)) return false;
    const bool whole = TW == Q;
    const int cs = whole ? 0 : (pw & 1);
    const int Wr = whole ? W + 2 * pw : (TW + S - 1 + cs + 1) & ~1;
    const int npairs = whole ? W / 2 : Wr / 2;
    const long PQv = (long)P * TW;
    const int rows_max = halo_rows_max(Mv, BN, PQv, TW, a.Hp, R);
    const size_t stage = (size_t)(BM * (2 * R * S + 1) + rows_max * 2 * Wr + 2) * 16;
    const size_t lds = a.stages * stage;
    if (lds > 160 * 1024 || 2 * ((rows_max * npairs + 255) / 256) > 8) return false;
    c = Cand{TW, WM, rows_max, Wr, 2 * Wr, 0, rows_max * 2 * Wr, lds, (long)nstrips * TW};
    return true;
  };
  Cand best{}, c{};
  bool have = false;
  auto better = [&](const Cand& x) {
    // (fits two per CU, fewer virtual columns, whole rows / wider strips)
    const bool x2 = x.lds <= 80 * 1024, b2 = best.lds <= 80 * 1024;
    if (!have) return true;
    if (x2 != b2) return x2;
    if (x.cols != best.cols) return x.cols < best.cols;
    // fewer staged input cells per block: less re-reading of halo rows
    return x.rows_max * x.Wp < best.rows_max * best.Wp;
  };
  const int tws[] = {Q, 128, 64, 32};
  for (int i = 0; i < 4; ++i) {
    const int TW = tws[i];
    if (i > 0 && TW >= Q) continue;
    if (eval(TW, 1, c) && better(c)) { best = c; have = true; }
    if (O > 64 && (!have || best.lds > 80 * 1024) && eval(TW, 2, c) && better(c)) { best = c; have = true; }
  }
  if (!have) return VH_ERR_UNSUPPORTED;
  // Row pitch: the 32 lanes of a fragment read consecutive positions, i.e.
  // consecutive 16-byte cells except at a row end, where the cell index jumps
  // by Wp - TW, and at an image end, by (Hp - P) Wp + Wp - TW + img_d.  With
  // both = 0 (mod 16) every 16 lanes that share a read cycle are on distinct
  // banks.  Taken when the larger stage keeps every decision the tight pitch
  // 2 Wr led to (blocks per CU, fused form's static stage size).
  {
    const int BMb = best.WM * fm * 32, BNb = (4 / best.WM) * 64;
    const long PQv = (long)P * best.TW;
    const int imgs = (int)((BNb - 1 + PQv - 1) / PQv) + 1;  // virtual images a block can span
    auto units = [&](int xc) { return BMb * (2 * R * S + 1) + xc + 2; };
    const bool two = best.lds <= 80 * 1024;
    const bool fused_base = units(best.xcells) <= kFusedStageUnits;
    const int wp = best.Wp + (((best.TW - best.Wp) % 16) + 16) % 16;
    const int d = (((-(a.Hp - P) * wp) % 16) + 16) % 16;
    const int xc = best.rows_max * wp + (imgs - 1) * d;
    const size_t lds_wp = (size_t)a.stages * units(xc) * 16;
    if (lds_wp <= (two ? 80 * 1024 : 160 * 1024) && !(fused_base && units(xc) > kFusedStageUnits)) {
      best.Wp = wp;
      best.img_d = d;
      best.xcells = xc;
      best.lds = lds_wp;
    }
  }
  const int WM = best.WM, rows_max = best.rows_max;
  a.TW = best.TW;
  a.nstrips = (Q + a.TW - 1) / a.TW;
  a.Wp = best.Wp;
  a.hoff = best.Wr;
  a.img_d = best.img_d;
  a.xcells = best.xcells;
  a.M = N * a.nstrips * P * a.TW;
  a.fPQ = FastDiv((uint32_t)(P * a.TW));
  a.fQ = FastDiv((uint32_t)a.TW);
  a.fStrips = FastDiv((uint32_t)a.nstrips);
  const bool whole = a.nstrips == 1;
  a.cs = whole ? 0 : (pw & 1);
  a.lcol0 = whole ? 0 : -pw - a.cs;
  a.lcell0 = whole ? pw : 0;
  // strips load the cells their taps read (the pitch may leave unused cells past them)
  a.npairs = whole ? W / 2 : ((a.TW + S - 1 + a.cs + 1) & ~1) / 2;
  a.fW2 = FastDiv((uint32_t)a.npairs);
  a.rows_max = rows_max;
  a.fRowsMax = FastDiv((uint32_t)rows_max);
  // vector epilogue: whole rows, runs of 8 positions inside one image, aligned
  // output (and mask); its LDS (4 waves x 64 x 72 bf16) reuses the stages
  a.vec_epi = (whole && (P * Q) % 8 == 0 && ((uintptr_t)y & 15) == 0 && (act != 2 || ((uintptr_t)mask & 15) == 0))
                  ? 1 : 0;
  // else the pair epilogue: even Q and strip width, 4-byte aligned output (and mask).
  // (Where both apply, the vector form measured 1-4 us faster on 64@56 and 128@28.)
  a.pair_epi = (!a.vec_epi && Q % 2 == 0 && a.TW % 2 == 0 && ((uintptr_t)y & 3) == 0 &&
                (act != 2 || ((uintptr_t)mask & 3) == 0))
                   ? 1 : 0;
  const int BMt = WM * fm * 32;
  const long tiles = ((long)a.M + (4 / WM) * 64 - 1) / ((4 / WM) * 64) * ((O + BMt - 1) / BMt);
  const int stage_units = BMt * (2 * R * S + 1) + a.xcells + 2;
  // Three blocks per CU with one LDS stage pays off for grids of many blocks
  // with several channel groups (one group is single-stage already).
  // Fused form (two register sets, whole channel groups, stages and the
  // vector epilogue within the static stage size): 3x3, 64 x 256 tiles with
  // at most 4 x items per thread.
  const bool fused_ok = fm == 2 && R == 3 && S == 3 && WM == 1 && nk >= 2 && C % 16 == 0 && halo_xi(a) <= 4 &&
                        stage_units <= kFusedStageUnits && (!a.vec_epi || 4 * 64 * 72 * 2 <= kFusedStageUnits * 16);
  // A forward over whole rows stays on the fused form, which reads W itself
  // (no relayout launch): 64@56, 1568 tiles, 51.7 -> 47.5 us a pass; the
  // input gradient and column strips measured faster three blocks per CU.
  const bool wpe3 = R == 3 && S == 3 && nk >= 2 && tiles >= VH_HALO_WPE3_MIN_TILES && halo_xi(a) <= (WM == 1 ? 4 : 2) &&
                    !(w_mode == 0 && whole && fused_ok);
  if (wpe3) a.stages = 1;
  const size_t lds_st = wpe3 ? best.lds / 2 : best.lds;
  const size_t lds = a.vec_epi ? std::max<size_t>(lds_st, 4 * 64 * 72 * 2) : lds_st;
  const bool fused = !wpe3 && fused_ok;
  // The fused forward reads W [O][C][3][3] directly (no relayout launch).  Each
  // block then repacks its weights itself: free in the fused form (128@28 and
  // 256@14 ran as fast as with the grouped copy), 4 us more than the relayout
  // saves in the three-blocks-per-CU form of 64@56 (1568 blocks, 9 scattered
  // 8-byte loads per lane and group), which keeps the grouped copy.
  const bool wd = w_mode == 0 && fused && (long)O * C * 18 < (1L << 31) - 16;
  if (wd) {
    a.wt = (const uint16_t*)w;
    a.w_bytes = O * C * 18;
  } else {
    VH_TRY_HALO(run_relayout_grouped(w, ws, O, C, R * S, w_mode, st));
  }
  if (wpe3) return pick_xi_wpe3(a, WM, fm, lds, st);
  if (fused) {
    if (wd)
      return halo_xi(a) <= 2 ? launch_halo<3, 3, 1, 2, VH_HALO_FUSED_WPE, true, true, VH_HALO_PC>(a, lds, st)
                             : launch_halo<3, 3, 1, 4, VH_HALO_FUSED_WPE, true, true, VH_HALO_PC>(a, lds, st);
    return halo_xi(a) <= 2 ? launch_halo<3, 3, 1, 2, VH_HALO_FUSED_WPE, true, false, VH_HALO_PC>(a, lds, st)
                           : launch_halo<3, 3, 1, 4, VH_HALO_FUSED_WPE, true, false, VH_HALO_PC>(a, lds, st);
  }
  if (fm == 1) return pick_xi<3, 3, 1, 1>(a, lds, st);
#define VH_HALO(RR, SS)                                           \
  if (R == RR && S == SS) {                                       \
    return WM == 2 ? pick_xi<RR, SS, 2>(a, lds, st) : pick_xi<RR, SS, 1>(a, lds, st); \
  }
  VH_HALO(3, 3)
  VH_HALO(5, 5)
  VH_HALO(1, 1)
#undef VH_HALO
  return VH_ERR_UNSUPPORTED;
}

}  // namespace vh
