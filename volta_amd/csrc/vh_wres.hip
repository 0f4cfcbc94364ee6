// vh_wres.hip -- bf16 3x3 stride-1 convolution for at most 64 input and 64
// output channels, gfx950 MFMA (v_mfma_f32_32x32x16_bf16), NCHW tensors.
//
// With C and O at most 64 the whole weight tensor (64 x C x 9 bf16, 73.7 KB at
// C = 64) fits in LDS beside the input staging, so a block keeps it resident
// and streams only x.  The grid is one block per CU (persistent): block b
// takes a contiguous range of 256-position tiles and runs them back to back.
//
// GEMM view as in the halo kernel: rows = output channels o, columns = output
// positions m = (n, p, q), K = (input channel c, tap r, tap s).  Per 16-channel
// group the producers stage the input "halo" of the tile -- every padded input
// row its 256 positions touch, channel-packed, cell = (ext row, padded column)
// -> 16 channels in two 8-channel half-planes -- and the consumers run all nine
// taps against it: tap (r, s) of position (n, p, q) is cell (n*Hp + p + r, q + s).
//
// Roles (512 threads, one block per CU, two waves per SIMD):
//   waves 0-3 (consumers): 64 o x 64 positions each (2 x 2 fragments of 32 x 32).
//     The fragment reads run two taps ahead of the MFMAs, across channel groups
//     and tiles, so that one wave per SIMD keeps the MFMA pipe fed.
//   waves 4-7 (producers): 16-byte loads (8 columns of a channel row), a quad
//     of lanes per 8 x 8 item transposing it into 8 channel-packed cells with
//     quad permutes; they run ahead across tile boundaries.
// Three LDS stages, one barrier per channel group: barrier G certifies that
// groups G and G+1 are staged and that the consumers are done with group G-1
// (whose stage then takes group G+2).
#include "vh_kernels.hpp"

namespace vh {

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32v2 __attribute__((vector_size(8)));  // the 64-bit buffer store's operand

struct WresArgs {
  const uint16_t* x;     // [N][C][H][W]
  const uint16_t* w;     // grouped: [nk][O][19][8] (units 2*tap, 2*tap+1 = channels 0-7, 8-15
                         // of the group, unit 18 zero); else W [O][C][3][3] with C % 16 == 0
  const uint16_t* bias;  // [O] or nullptr
  const uint16_t* mask;  // act 2: [N][O][P][Q]
  uint16_t* y;           // [N][O][P][Q]
  int N, C, H, W, O, P, Q, ph, pw;
  int Hp, Wp;            // ext rows per image (H + 2 ph); LDS cells per ext row (>= W + 2 pw)
  int nk;                // channel groups: ceil(C / 16)
  int M;                 // N*P*Q positions
  int tiles;             // ceil(M / 256)
  int rows_max;          // most ext rows any tile spans
  int nocts;             // 8-column octets per input row: W / 8
  int nitems;            // load items per group: 2 half-planes x rows_max x nocts
  int x_bytes, y_bytes, w_bytes;
  int grouped;           // 1: w is the grouped copy
  FastDiv fPQ, fQ, fHp, fOct, fRows;  // P*Q, Q, Hp, nocts, rows_max
};

constexpr int kWpu = 19;                 // 16-byte units per output channel and group
constexpr int kBM = 64, kBN = 256;       // tile: 64 output channels x 256 positions
constexpr int kWUnits = kBM * kWpu;      // units per group of the resident weights
constexpr int kStages = 3;

__device__ __forceinline__ uint32_t perm_b32(uint32_t s0, uint32_t s1, uint32_t sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}
// value of lane ^ 1 and lane ^ 2 (quad permutes, DPP)
__device__ __forceinline__ uint32_t xor1(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t xor2(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
}
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
// two floats -> packed bf16 (lo, hi), one v_cvt_pk_bf16_f32 (round to nearest even)
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const f32x2v f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2v));
}

template <int XR, int ACT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void conv_wres_bf16_kernel(WresArgs a) {
  extern __shared__ __attribute__((aligned(16))) u32x4 lds[];

  const int wave_all = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const bool producer = wave_all >= 4;
  const int tid = (int)threadIdx.x & 255, lane = tid & 63;
  const int wave = wave_all & 3;

  // Tiles of this block: tb, tb + T, tb + 2T, ... (T = grid size).  tb =
  // xcd_block(T): the blocks running at the same time on one XCD take
  // neighbouring tiles, whose shared halo rows then come from that XCD's L2.
  const int T = (int)gridDim.x;
  const int tb = xcd_block(T);
  const int nt = tb < a.tiles ? (a.tiles - tb + T - 1) / T : 0;
  const int TG = nt * a.nk;  // channel groups this block runs
  if (TG == 0) return;

  const int Wp = a.Wp;
  const int cells = a.rows_max * Wp;      // cells per half-plane
  const int stage_units = 2 * cells + 1;  // the last unit: sink for unused load items
  u32x4* const wl = lds;                  // resident weights: [g][o][19]
  u32x4* const xs0 = lds + a.nk * kWUnits;

  // ---- resident weights (all 512 threads; the producers first issue their
  // loads of the first two channel groups, so that both fetches overlap) ----
  auto load_weights = [&]() {
    const __amdgpu_buffer_rsrc_t wrsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, a.w_bytes, 0x00020000);
    if (a.grouped) {
      // unit q of [g][o][19]: (g*O + o)*19 + u of the copy; rows past O read zeros
      const int total = a.nk * kWUnits;
      u32x4 v[10];
#pragma unroll
      for (int k = 0; k < 10; ++k) {
        const int q = (int)threadIdx.x + k * 512;
        const int g = q / kWUnits, r = q - g * kWUnits, o = r / kWpu, u = r - o * kWpu;
        const int off = q < total && o < a.O ? ((g * a.O + o) * kWpu + u) * 16 : (int)0x80000000u;
        v[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, off, 0, 0));
      }
#pragma unroll
      for (int k = 0; k < 10; ++k) {
        const int q = (int)threadIdx.x + k * 512;
        if (q < total) wl[q] = v[k];
      }
    } else if ((int)threadIdx.x < a.nk * 128) {
      // thread -> (group g, output channel o, half h): the 8 channels x 9 taps of
      // W[o][16g + 8h .. +7][*] are 72 contiguous bf16 (144 bytes, 16-byte
      // aligned), loaded as 9 x 16 bytes and repacked into the 9 units of the taps
      const int t = (int)threadIdx.x, g = t >> 7, o = (t >> 1) & 63, h = t & 1;
      const int off = o < a.O ? (o * a.C + g * 16 + h * 8) * 18 : (int)0x80000000u;
      uint32_t d[36];
#pragma unroll
      for (int k = 0; k < 9; ++k) {
        const u32x4 q = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, off + 16 * k, 0, 0));
        d[4 * k] = q.x; d[4 * k + 1] = q.y; d[4 * k + 2] = q.z; d[4 * k + 3] = q.w;
      }
      // element e = c*9 + tap sits in dword e/2, half e%2; the unit of tap tp takes
      // elements tp, 9+tp, ..., 63+tp (channels 0..7)
      auto el2 = [&](int e0, int e1) {  // bf16 e0 low, e1 high
        const uint32_t sel = (2u * (e0 & 1)) | ((2u * (e0 & 1) + 1u) << 8) | ((4u + 2u * (e1 & 1)) << 16) |
                             ((5u + 2u * (e1 & 1)) << 24);
        return perm_b32(d[e1 >> 1], d[e0 >> 1], sel);
      };
      u32x4* dst = wl + (g * kBM + o) * kWpu + h;
#pragma unroll
      for (int tp = 0; tp < 9; ++tp) {
        u32x4 u;
        u.x = el2(tp, 9 + tp);
        u.y = el2(18 + tp, 27 + tp);
        u.z = el2(36 + tp, 45 + tp);
        u.w = el2(54 + tp, 63 + tp);
        dst[2 * tp] = u;
      }
    }
  };

  if (producer) {
    // ---- producers: x staging ----
    const int HW = a.H * a.W, HW2 = HW * 2;
    const __amdgpu_buffer_rsrc_t xrsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.x_bytes, 0x00020000);
    // Load items: item i = (half-plane, ext row e, octet oc) = 8 columns x 8
    // channels, served by a quad of lanes (item k*64 + tid/4 of round k): lane t
    // = tid % 4 loads 16 bytes of channels t and t+4 of the half-plane, the quad
    // transposes the 8 x 8 block (rows of channel t+4h in register h; the
    // exchange between rows t and t+4 is a renaming, the other two stages quad
    // permutes), and lane t stores the cells of columns t and t+4.  The LDS cell
    // is the same for every tile (items past a tile's rows store into cells its
    // taps never read); items past the last go to the sink.
    const int qt = tid & 3;
    int x_lofs[XR], x_e[XR], x_oc[XR], x_half[XR];
#pragma unroll
    for (int k = 0; k < XR; ++k) {
      const int i = k * 64 + (tid >> 2);
      int half = 0, e = -1, oc = 0;
      if (i < a.nitems) {
        const int per_half = a.rows_max * a.nocts;
        half = i >= per_half ? 1 : 0;
        uint32_t ee, oo;
        a.fOct.divmod((uint32_t)(i - half * per_half), ee, oo);
        e = (int)ee;
        oc = (int)oo;
      }
      x_e[k] = e;
      x_oc[k] = oc;
      x_half[k] = half;
      // byte offset of column t's cell in a stage (sink: 16 bytes past the two half-planes)
      x_lofs[k] = (e >= 0 ? half * cells + e * Wp + a.pw + 8 * oc + qt : 2 * cells) * 16;
    }
    int x_voff[XR];
    auto tile_offsets = [&](int t) {
      uint32_t n_a, pq_a, p_a, q_a, n_b, pq_b, p_b, q_b;
      const int m0 = t * kBN, ml = min(m0 + kBN, a.M) - 1;
      a.fPQ.divmod((uint32_t)m0, n_a, pq_a);
      a.fQ.divmod(pq_a, p_a, q_a);
      a.fPQ.divmod((uint32_t)ml, n_b, pq_b);
      a.fQ.divmod(pq_b, p_b, q_b);
      const int e_start = (int)n_a * a.Hp + (int)p_a;
      const int rows = (int)n_b * a.Hp + (int)p_b + 3 - e_start;
#pragma unroll
      for (int k = 0; k < XR; ++k) {
        int voff = (int)0x80000000u;
        if (x_e[k] >= 0 && x_e[k] < rows) {
          uint32_t n, hr;
          a.fHp.divmod((uint32_t)(e_start + x_e[k]), n, hr);
          const int h = (int)hr - a.ph;
          if (h >= 0 && h < a.H) voff = (((int)n * a.C + x_half[k] * 8 + qt) * HW + h * a.W + 8 * x_oc[k]) * 2;
        }
        x_voff[k] = voff;
      }
    };
    u32x4 xreg[2][XR][2];
    // (tile, group) of the next group to load, advanced by one per prep (no
    // division); c0 and crem: its channel offset and the channels left from it
    // (zeros past C and past the last group)
    int lt = tb, lg = 0, lG = 0, c0 = 0, crem = 0;
    auto prep = [&]() {
      const bool live = lG < TG;
      if (live && lg == 0) tile_offsets(lt);
      c0 = lg * 16;
      crem = live ? a.C - c0 : 0;
      ++lG;
      if (++lg == a.nk) {
        lg = 0;
        lt += T;
      }
    };
    // rounds past the last item of this wave are skipped (wave-uniform)
    const int wave_items = a.nitems - wave * 16;
    auto gload = [&](auto SET) {
      constexpr int sI = decltype(SET)::value;
#pragma unroll
      for (int k = 0; k < XR; ++k) {
        if (k * 64 < wave_items) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            // channel c0 + 8*half + t + 4h of the half-plane (half and t in x_voff)
            const int off = x_half[k] * 8 + qt + 4 * h < crem ? x_voff[k] : (int)0x80000000u;
            xreg[sI][k][h] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrsrc, off, (c0 + 4 * h) * HW2, 0));
          }
        }
      }
    };
    const bool b1 = qt & 1, b2 = qt & 2;
    const uint32_t sp = b1 ? 0x05040100u : 0x07060302u;  // lane ^ 1 stage: lo / hi halves of (d0, d1)
    const uint32_t sa = b1 ? 0x03020504u : 0x05040100u;
    const uint32_t sb = b1 ? 0x03020706u : 0x07060100u;
    auto sstore = [&](auto SET, int st) {
      constexpr int sI = decltype(SET)::value;
      char* base = reinterpret_cast<char*>(xs0 + st * stage_units);
#pragma unroll
      for (int k = 0; k < XR; ++k) {
        if (k * 64 < wave_items) {
          // virtual lane r = t + 4h holds row r; stage lane ^ 4 is in-register:
          // row t keeps columns 0-3 and takes columns 0-3 of row t+4 (and so on)
          const u32x4 R0 = xreg[sI][k][0], R1 = xreg[sI][k][1];
          u32x4 d[2];
          d[0] = u32x4{R0.x, R0.y, R1.x, R1.y};
          d[1] = u32x4{R0.z, R0.w, R1.z, R1.w};
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            u32x4& v = d[h];
            {  // lane ^ 2: dwords 1, 3 (t & 2 == 0) or 0, 2
              const uint32_t r0 = xor2(b2 ? v.x : v.y), r1 = xor2(b2 ? v.z : v.w);
              if (b2) { v.x = r0; v.z = r1; } else { v.y = r0; v.w = r1; }
            }
            {  // lane ^ 1: the odd elements (t even) or the even ones, packed two per dword
              const uint32_t s0 = perm_b32(v.y, v.x, sp), s1 = perm_b32(v.w, v.z, sp);
              const uint32_t r0 = xor1(s0), r1 = xor1(s1);
              v.x = perm_b32(r0, v.x, sa);
              v.y = perm_b32(r0, v.y, sb);
              v.z = perm_b32(r1, v.z, sa);
              v.w = perm_b32(r1, v.w, sb);
            }
            // column t + 4h of the octet (both to the sink for items past the last)
            *reinterpret_cast<u32x4*>(base + x_lofs[k] + (x_e[k] >= 0 ? h * 64 : 0)) = v;
          }
        }
      }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // register set G & 1 holds group G; group G goes to stage G % 3
    prep();
    gload(I0{});
    prep();
    gload(I1{});
    load_weights();
    // padding cells of every stage, zeroed once (never written by the loader):
    // per (stage, half-plane, ext row) the cells [0, pw) and [W + pw, Wp)
    {
      const u32x4 z = {0u, 0u, 0u, 0u};
      const int padc = Wp - a.W;
      for (int i = tid; i < 2 * kStages * a.rows_max; i += 256) {
        uint32_t sh, e;
        a.fRows.divmod((uint32_t)i, sh, e);
        u32x4* rowp = xs0 + (sh >> 1) * stage_units + (sh & 1) * cells + e * Wp;
        for (int pc = 0; pc < padc; ++pc) rowp[pc < a.pw ? pc : a.W + pc] = z;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    prep();
    sstore(I0{}, 0);
    gload(I0{});
    prep();
    if (TG > 1) sstore(I1{}, 1);
    gload(I1{});
    __syncthreads();  // barrier 0: weights and groups 0, 1 staged
    int st = 2;       // stage of group G + 2
    for (int G = 0; G + 1 < TG; G += 2) {
      // group G+2 (set 0) into the stage of group G-1, then group G+3 (set 1)
      prep();  // group G+4
      if (G + 2 < TG) sstore(I0{}, st);
      gload(I0{});
      st = st == 2 ? 0 : st + 1;
      __syncthreads();
      if (G + 2 >= TG) break;
      prep();  // group G+5
      if (G + 3 < TG) sstore(I1{}, st);
      gload(I1{});
      st = st == 2 ? 0 : st + 1;
      __syncthreads();
    }
    return;
  }

  // ---- consumers ----
  load_weights();
  const int wn = wave * 64;  // wave's first position in the tile
  const int half_l = lane >> 5, row_l = lane & 31;
  const int PQ = a.P * a.Q, PQ2 = PQ * 2;
  // fp32 bias of the accumulator rows of this lane (o = i*32 + (v>>2)*8 + (lane>>5)*4 + (v&3)),
  // loaded once: the accumulators of every tile start from it (act 2, the input
  // gradient, has no bias)
  constexpr bool kBias = ACT != 2;
  float bv[2][16];
  if constexpr (kBias) {
    const __amdgpu_buffer_rsrc_t brsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.bias, (short)0, a.bias ? a.O * 2 : 0, 0x00020000);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        bv[i][v] = bf16_to_f32((uint16_t)__builtin_amdgcn_raw_buffer_load_b16(
            brsrc, (i * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3)) * 2, 0, 0));
  }
  const __amdgpu_buffer_rsrc_t yrsrc = __builtin_amdgcn_make_buffer_rsrc((void*)a.y, (short)0, a.y_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t mrsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)(ACT == 2 ? a.mask : a.y), (short)0, ACT == 2 ? a.y_bytes : 0,
                                        0x00020000);
  const bool full_o = a.O >= kBM;
  // LDS cell offset of each B-fragment column (positions of the tile, relative
  // to the tile's first ext row); 0 for positions past M
  auto tile_bcell = [&](int t, int (&bc)[2]) {
    const int m0 = t * kBN;
    uint32_t n_a, pq_a, p_a, q_a;
    a.fPQ.divmod((uint32_t)min(m0, a.M - 1), n_a, pq_a);
    a.fQ.divmod(pq_a, p_a, q_a);
    const int e_start = (int)n_a * a.Hp + (int)p_a;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int m = m0 + wn + j * 32 + row_l;
      int cidx = 0;
      if (m < a.M) {
        uint32_t n, pq, p, q;
        a.fPQ.divmod((uint32_t)m, n, pq);
        a.fQ.divmod(pq, p, q);
        cidx = ((int)n * a.Hp + (int)p - e_start) * Wp + (int)q;
      }
      bc[j] = cidx;
    }
  };
  const u32x4* const xsb = lds + a.nk * kWUnits + half_l * cells;
  const u32x4* const wsb = lds + row_l * kWpu + half_l;
  bf16x8 fa[3][2], fb[3][2];  // fragments of three taps in flight (slot = tap % 3)
  // fragments of tap `tap` of channel group g from stage st, columns bc
  auto rd = [&](int slot, int g, int st, const int (&bc)[2], int tap) {
    const int r = tap / 3, s = tap - r * 3;
    const u32x4* W_ = wsb + g * kWUnits + tap * 2;
    const u32x4* X_ = xsb + st * stage_units + r * Wp + s;
#pragma unroll
    for (int i = 0; i < 2; ++i) fa[slot][i] = __builtin_bit_cast(bf16x8, W_[i * 32 * kWpu]);
#pragma unroll
    for (int j = 0; j < 2; ++j) fb[slot][j] = __builtin_bit_cast(bf16x8, X_[bc[j]]);
  };
  // Epilogue pieces: rows 4b .. 4b+3 (+4 in the upper half-wave) of fragment
  // (i, j) of a finished tile, as packed bf16 pairs pk (rows 4b, 4b+1 and 4b+2,
  // 4b+3 at the lane's position).  A 4 x 4 transpose in each quad (lane p = lane
  // & 3 holds position p) leaves row p of the quad's 4 positions in lane p: one
  // 8-byte store.  yp: the quad's y offset, out of range when there is nothing to store.
  const int qp = lane & 3;
  const uint32_t tsel = (qp & 1) ? 0x03020706u : 0x05040100u;
  uint32_t pk[2][2][8];
  u32x2 mkp[2][2][4];
  int yp[2] = {(int)0x80000000u, (int)0x80000000u};
  auto epi_piece = [&](int i, int j, int b) {
    const uint32_t d0 = pk[i][j][2 * b], d1 = pk[i][j][2 * b + 1];
    // lane ^ 2: positions p, p^2 of rows (0,1) (p < 2) or (2,3)
    const uint32_t r = xor2((qp & 2) ? d0 : d1);
    const uint32_t A = (qp & 2) ? r : d0, B = (qp & 2) ? d1 : r;
    // lane ^ 1: the row of this lane at positions 0, 1 and 2, 3
    const uint32_t rA = xor1(A), rB = xor1(B);
    u32x2 o;
    o.x = perm_b32(rA, A, tsel);
    o.y = perm_b32(rB, B, tsel);
    if constexpr (ACT == 2) {
      const u32x2 m = mkp[i][j][b];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t mm = h ? m.y : m.x;
        const uint32_t keep = (bf16_to_f32((uint16_t)(mm & 0xffffu)) > 0.f ? 0x0000ffffu : 0u) |
                              (bf16_to_f32((uint16_t)(mm >> 16)) > 0.f ? 0xffff0000u : 0u);
        if (h) o.y &= keep; else o.x &= keep;
      }
    }
    const int orow = i * 32 + b * 8;  // wave-uniform part of the row
    if (full_o || orow + (lane >> 5) * 4 + qp < a.O)
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32v2, o), yrsrc,
                                            (int)((uint32_t)yp[j] + (uint32_t)(orow * PQ2)), 0, 0);
  };

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int u = 0; u < 8; ++u) pk[i][j][u] = 0u;
#pragma unroll
      for (int b = 0; b < 4; ++b) mkp[i][j][b] = u32x2{0u, 0u};
    }
  int bc[2], bn[2];
  tile_bcell(tb, bc);
  __syncthreads();  // barrier 0
  rd(0, 0, 0, bc, 0);
  rd(1, 0, 0, bc, 1);
  int G = 0, sc = 0;  // block-local group, its stage
  using E0 = std::integral_constant<int, 0>;
  using E1 = std::integral_constant<int, 1>;
  f32x16 acc[2][2];
  u32x2 mk[2][2][4];
  int yq[2];
  // one channel group g of the current tile: nine taps, the fragment reads two
  // taps ahead; EPI: the previous tile's epilogue pieces placed between the MFMAs
  auto group = [&](int g, auto EPI) {
    constexpr bool epi = decltype(EPI)::value;
    const bool lastg = g == a.nk - 1;
    const int gn = lastg ? 0 : g + 1;
    const int sn = sc == 2 ? 0 : sc + 1;
    int bx[2];
    bx[0] = lastg ? bn[0] : bc[0];
    bx[1] = lastg ? bn[1] : bc[1];
    if (ACT == 2 && lastg) {
      // the ReLU-backward mask of this tile's output, loaded before its last products
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            mk[i][j][b] = __builtin_bit_cast(
                u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                           mrsrc, (int)((uint32_t)yq[j] + (uint32_t)((i * 32 + b * 8) * PQ2)), 0, 0));
    }
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      // fragments of the tap after next (taps 7, 8: the next group's taps 0, 1)
      if (tap + 2 < 9) rd((tap + 2) % 3, g, sc, bc, tap + 2);
      else rd((tap + 2) % 3, gn, sn, bx, tap + 2 - 9);
      const int sl = tap % 3;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[sl][i], fb[sl][j], acc[i][j], 0, 0, 0);
      if constexpr (epi) {
        // taps 0..7: two epilogue pieces each (16 in all)
        if (tap < 8) {
          epi_piece(tap >> 2, (tap >> 1) & 1, (tap & 1) * 2);
          epi_piece(tap >> 2, (tap >> 1) & 1, (tap & 1) * 2 + 1);
        }
      }
    }
    // per tap: one fragment read between consecutive MFMAs (EPI: and the
    // epilogue's VALU work and stores after each MFMA)
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (epi && tap < 8) {
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
          if (k & 1) __builtin_amdgcn_sched_group_barrier(0x040, 1, 0);
        }
      }
    }
    sc = sn;
    if (G + 1 < TG) __syncthreads();  // barrier G+1
    ++G;
  };
  for (int t = tb; t < a.tiles; t += T) {
    tile_bcell(t + T, bn);
    // y offset of this lane's quad (positions m .. m+3, m = 0 mod 4; Q = 0 mod 4
    // keeps them in one image row) at row (lane>>5)*4 + (lane&3); out of range past M
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t mq = (uint32_t)(t * kBN + wn + j * 32 + (lane & 28));
      uint32_t n, pq;
      a.fPQ.divmod(mq, n, pq);
      yq[j] = (int)mq < a.M ? (int)((n * (uint32_t)a.O * (uint32_t)PQ + pq) * 2u) + ((lane >> 5) * 4 + qp) * PQ2
                            : (int)0x80000000u;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = kBias ? bv[i][v] : 0.f;
    group(0, E1{});  // with the previous tile's epilogue (nothing stored before the first)
    for (int g = 1; g < a.nk; ++g) group(g, E0{});
    bc[0] = bn[0];
    bc[1] = bn[1];
    // this tile's results: activation, one rounding to bf16; stored during the next tile
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          float x0 = acc[i][j][2 * u], x1 = acc[i][j][2 * u + 1];
          if (ACT == 1) {
            x0 = fmaxf(x0, 0.f);
            x1 = fmaxf(x1, 0.f);
          }
          pk[i][j][u] = pack_bf16(x0, x1);
        }
    if constexpr (ACT == 2) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int b = 0; b < 4; ++b) mkp[i][j][b] = mk[i][j][b];
    }
    yp[0] = yq[0];
    yp[1] = yq[1];
  }
  // the last tile's epilogue
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int b = 0; b < 4; ++b) epi_piece(i, j, b);
}

int cu_count() {
  static int n = 0;
  static std::once_flag once;
  std::call_once(once, [] {
    int dev = 0, c = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) ==
                                                 hipSuccess && c > 0)
      n = c;
    else
      n = 256;
  });
  return n;
}

size_t wres_lds_bytes(int rows_max, int Wp, int nk) {
  return (size_t)(nk * kWUnits + kStages * (2 * rows_max * Wp + 1)) * 16;
}

}  // namespace

int wres_conv_bf16(const void* x, const void* w, int w_mode, void* ws, const void* bias, void* y, int N, int C,
                   int H, int W, int O, int ph, int pw, hipStream_t st, int act, const void* mask) {
  const int P = H + 2 * ph - 2, Q = W + 2 * pw - 2;
  if (C < 1 || C > 64 || O < 1 || O > 64 || P <= 0 || Q <= 0 || ph > 2 || pw > 2) return VH_ERR_UNSUPPORTED;
  // 16-byte row loads (W % 8) and 4-position output stores (Q % 4, 8-byte aligned y / mask)
  if ((W % 8) != 0 || (Q % 4) != 0 || act < 0 || act > 2 || (act == 2 && bias)) return VH_ERR_UNSUPPORTED;
  if (((uintptr_t)x & 15) != 0 || ((uintptr_t)y & 7) != 0 || (act == 2 && ((uintptr_t)mask & 7) != 0))
    return VH_ERR_UNSUPPORTED;
  const long xb = (long)N * C * H * W * 2, yb = (long)N * O * P * Q * 2;
  if (xb >= (1L << 31) - 16 || yb >= (1L << 31) - 16 || (long)N * P * Q >= (1L << 31) - (1L << 17)) return VH_ERR_UNSUPPORTED;
  // the forward with whole 16-channel groups reads W itself; otherwise the grouped copy
  const int grouped = !(w_mode == 0 && C % 16 == 0);
  WresArgs a;
  a.x = (const uint16_t*)x;
  a.w = (const uint16_t*)w;
  a.bias = (const uint16_t*)bias;
  a.mask = (const uint16_t*)mask;
  a.y = (uint16_t*)y;
  a.N = N; a.C = C; a.H = H; a.W = W; a.O = O; a.P = P; a.Q = Q; a.ph = ph; a.pw = pw;
  a.Hp = H + 2 * ph;
  a.nk = (C + 15) / 16;
  a.M = N * P * Q;
  a.tiles = (a.M + kBN - 1) / kBN;
  a.rows_max = halo_rows_max(a.M, kBN, (long)P * Q, Q, a.Hp, 3);
  a.nocts = W / 8;
  a.nitems = 2 * a.rows_max * a.nocts;
  a.x_bytes = (int)xb;
  a.y_bytes = (int)yb;
  a.w_bytes = grouped ? a.nk * O * kWpu * 16 : O * C * 18;
  a.grouped = grouped;
  a.fPQ = FastDiv((uint32_t)(P * Q));
  a.fQ = FastDiv((uint32_t)Q);
  a.fHp = FastDiv((uint32_t)a.Hp);
  a.fOct = FastDiv((uint32_t)a.nocts);
  a.fRows = FastDiv((uint32_t)a.rows_max);
  // Row pitch: 32 lanes of a fragment read consecutive positions, i.e.
  // consecutive cells except at a row end, where the index jumps by Wp - Q.
  // Wp = Q (mod 16) keeps every 16 lanes on distinct banks; kept where LDS allows.
  const int wp0 = W + 2 * pw;
  a.Wp = wp0 + ((Q - wp0) % 16 + 16) % 16;
  if (wres_lds_bytes(a.rows_max, a.Wp, a.nk) > 160 * 1024) a.Wp = wp0;
  const size_t lds = wres_lds_bytes(a.rows_max, a.Wp, a.nk);
  if (lds > 160 * 1024) return VH_ERR_UNSUPPORTED;
  const int xr = (a.nitems + 63) / 64;  // load rounds per group: 64 items per round
  if (xr > 8) return VH_ERR_UNSUPPORTED;
  if (grouped) {
    const int r = run_relayout_grouped(w, ws, O, C, 9, w_mode, st);
    if (r != VH_OK) return r;
    a.w = (const uint16_t*)ws;
  }
  const int grid = std::min(a.tiles, cu_count());
#define VH_WRES(XRV, ACTV)                                                         \
  do {                                                                             \
    auto k = conv_wres_bf16_kernel<XRV, ACTV>;                                     \
    VH_LDS_LIMIT_ONCE(k);                                                          \
    k<<<dim3((unsigned)grid), 512, lds, st>>>(a);                                  \
  } while (0)
#define VH_WRES_ACT(XRV)                    \
  do {                                      \
    if (act == 0) VH_WRES(XRV, 0);          \
    else if (act == 1) VH_WRES(XRV, 1);     \
    else VH_WRES(XRV, 2);                   \
  } while (0)
  if (xr <= 2) VH_WRES_ACT(2);
  else if (xr <= 3) VH_WRES_ACT(3);
  else if (xr <= 4) VH_WRES_ACT(4);
  else if (xr <= 6) VH_WRES_ACT(6);
  else VH_WRES_ACT(8);
#undef VH_WRES_ACT
#undef VH_WRES
  VH_LAUNCH_CHECK();
  return VH_OK;
}

}  // namespace vh
