// vh_common.hpp -- shared device/host helpers for libvolta_hip (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>

#include "../../include/volta_hip.h"

namespace vh {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;

// bf16 is carried as raw uint16_t bits in memory.
struct bf16 {
  uint16_t bits;
};

__host__ __device__ inline float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// Round-to-nearest-even, NaN kept quiet (same rule as half::bf16::from_f32).
// On the device this is gfx950's v_cvt_pk_bf16_f32 (RNE in hardware).
__host__ __device__ inline uint16_t f32_to_bf16(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint16_t, (__bf16)f);
#endif
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <typename T> struct Elem;
template <> struct Elem<float> {
  using storage = float;
  static constexpr int vec = 4;  // elements per 16-byte unit
  __device__ static inline float to_f32(float v) { return v; }
  __device__ static inline float from_f32(float v) { return v; }
};
template <> struct Elem<bf16> {
  using storage = uint16_t;
  static constexpr int vec = 8;
  __device__ static inline float to_f32(uint16_t v) { return bf16_to_f32(v); }
  __device__ static inline uint16_t from_f32(float v) { return f32_to_bf16(v); }
};

// Division by a runtime constant via multiply-high (Granlund-Montgomery,
// round-up variant). Valid for numerators < 2^31 and divisors in [1, 2^31).
struct FastDiv {
  uint32_t d, m, s;
  FastDiv() : d(1), m(0), s(0) {}
  explicit FastDiv(uint32_t div) : d(div) {
    s = 0;
    while ((1u << s) < div) ++s;
    uint64_t one = 1;
    m = (uint32_t)(((one << 32) * ((one << s) - div)) / div + 1);
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    uint32_t t = __umulhi(n, m);
    return (t + n) >> s;
  }
  __device__ __forceinline__ void divmod(uint32_t n, uint32_t& q, uint32_t& r) const {
    q = div(n);
    r = n - q * d;
  }
};

// XCD-aware block order.  The dispatcher deals the workgroups of a 1-D grid
// to the 8 XCDs (each with its own L2) round robin by block id.  Logical
// block L = xcd * (nb / 8) + slot puts consecutive logical blocks -- which
// the callers arrange to share input data -- on the same XCD.  Identity when
// nb is not a multiple of 8.  xcd_map applies the same order to block h of a
// group of nb blocks inside a larger grid (the group starting at a multiple of
// 8, so that h & 7 is still the XCD).
__device__ __forceinline__ int xcd_map(int h, int nb) {
  if (nb & 7) return h;
  return (h & 7) * (nb >> 3) + (h >> 3);
}
__device__ __forceinline__ int xcd_block(int nb) { return xcd_map(blockIdx.x, nb); }

// Global -> LDS copy of 16 bytes per lane without registers
// (buffer_load_dwordx4 ... lds): lane l's 16 bytes at buffer offset voff + soff
// land at LDS byte la + 16 l (lanes off in EXEC copy nothing; an out-of-range
// voff writes zeros).  M0 holds la (the s_nop covers the M0 -> LDS DMA
// hazard).  Inline assembly, so the compiler's wait-count pass does not track
// these copies: the caller waits for them itself (s_waitcnt vmcnt) before a
// barrier, and keeps M0 free of other uses in its kernel.
__device__ __forceinline__ void lds_copy16(__amdgpu_buffer_rsrc_t r, int voff, int soff, uint32_t la) {
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(r), "s"(soff), "s"(la)
               : "memory", "m0");
}

// s_waitcnt vmcnt(N) (N < 64), other counters untouched
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xf00);
}

// LDS byte address of a shared-memory pointer, wave-uniform
template <typename T>
__device__ __forceinline__ uint32_t lds_byte_addr(const T* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) T*)p);
}

// Deterministic reduction of split-K partial sums part[z][i] (z < splits,
// i < total) by a 256-thread block: 64 consecutive outputs per pass, wave w
// adds z = w, w+4, w+8, ... in order and the four wave sums are added in wave
// order.  Every load of a wave covers 64 consecutive floats of one slab.
// store(i, sum) writes the result.
template <typename Store>
__device__ __forceinline__ void reduce_splits_block(const float* __restrict__ part, int splits, long total,
                                                    Store store, int blk, int nblk) {
  __shared__ float red[4][64];
  const int j = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (long base = (long)blk * 64; base < total; base += (long)nblk * 64) {
    const long i = base + j;
    float s = 0.f;
    if (i < total) {
#pragma unroll 4
      for (int z = w; z < splits; z += 4) s += part[(size_t)z * total + i];
    }
    red[w][j] = s;
    __syncthreads();
    if (w == 0 && i < total) store(i, ((red[0][j] + red[1][j]) + red[2][j]) + red[3][j]);
    __syncthreads();
  }
}

template <typename Store>
__device__ __forceinline__ void reduce_splits_block(const float* __restrict__ part, int splits, long total,
                                                    Store store) {
  reduce_splits_block(part, splits, total, store, (int)blockIdx.x, (int)gridDim.x);
}

inline int reduce_splits_grid(long total) { return (int)std::min<long>((total + 63) / 64, 1L << 20); }

// The same reduction read as float4 quads (total % 4 == 0, 16-byte aligned
// slabs), for few outputs and many splits: a pass covers QB = 256 >> lg_g
// quads; the threads form G = 2^lg_g split groups (thread t: quad t % QB,
// group t / QB), group g adds z = g, g + G, ... in order with several 16-byte
// loads in flight per lane, and the G group sums are added in group order.
// store(i, sum) is called for each of the four outputs of a quad.
template <typename Store>
__device__ __forceinline__ void reduce_splits_vec4_block(const float* __restrict__ part, int splits, long total,
                                                         int lg_g, Store store, int blk, int nblk) {
  __shared__ float4 red4[256];
  const int t = threadIdx.x, G = 1 << lg_g, QB = 256 >> lg_g;
  const int q = t & (QB - 1), g = t >> (8 - lg_g);
  const long nq = total >> 2;
  const float4* p4 = reinterpret_cast<const float4*>(part);
  for (long base = (long)blk * QB; base < nq; base += (long)nblk * QB) {
    const long qi = base + q;
    float4 a = {0.f, 0.f, 0.f, 0.f};
    if (qi < nq) {
#pragma unroll 8
      for (int z = g; z < splits; z += G) {
        const float4 v = p4[(size_t)z * nq + qi];
        a.x += v.x; a.y += v.y; a.z += v.z; a.w += v.w;
      }
    }
    red4[t] = a;
    __syncthreads();
    if (g == 0 && qi < nq) {
      float4 r = red4[q];
      for (int h = 1; h < G; ++h) {
        const float4 v = red4[h * QB + q];
        r.x += v.x; r.y += v.y; r.z += v.z; r.w += v.w;
      }
      store(qi * 4 + 0, r.x);
      store(qi * 4 + 1, r.y);
      store(qi * 4 + 2, r.z);
      store(qi * 4 + 3, r.w);
    }
    __syncthreads();
  }
}

// Split groups for reduce_splits_vec4_block: about 8 loads per lane, at most 16 groups.
inline int reduce_vec4_lg_groups(int splits) {
  int lg_g = 0;
  while (lg_g < 4 && (splits >> (lg_g + 1)) >= 8) ++lg_g;
  return lg_g;
}
inline int reduce_vec4_grid(long total, int lg_g) {
  const long qb = 256 >> lg_g;
  return (int)std::min<long>((total / 4 + qb - 1) / qb, 1L << 20);
}

// Column-sum ownership on BN-column tiles of a product whose column tile is
// shared by tiles_m blocks: 2^cs_shift groups of 4 columns per block, the
// smallest power-of-2 width >= BN / tiles_m (at least 16 columns).
inline int colsum_shift(int tiles_m, int BN) {
  int w = 16;
  while (w < BN && w * tiles_m < BN) w <<= 1;
  int sh = 0;
  while ((4 << sh) < w) ++sh;
  return sh;
}

// Raises a kernel's dynamic-LDS limit to the CU's 160 KB.  Each call site is
// one template instantiation, so the flag is per kernel; std::call_once makes
// concurrent first launches from several host threads safe.
#define VH_LDS_LIMIT_ONCE(kern)                                                                        \
  do {                                                                                                 \
    static std::once_flag _vh_lds_once;                                                                \
    std::call_once(_vh_lds_once, [&] {                                                                 \
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),                                   \
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);               \
    });                                                                                                \
  } while (0)

// Record an error message for vh_last_error(); returns the status.
int set_error(int status, const char* fmt, ...);

}  // namespace vh

#define VH_HIP_CHECK(expr)                                                          \
  do {                                                                              \
    hipError_t _e = (expr);                                                         \
    if (_e != hipSuccess)                                                           \
      return ::vh::set_error(_e == hipErrorOutOfMemory ? VH_ERR_OOM : VH_ERR_LAUNCH, \
                             "%s failed: %s", #expr, hipGetErrorString(_e));        \
  } while (0)

#define VH_LAUNCH_CHECK()                                                           \
  do {                                                                              \
    hipError_t _e = hipGetLastError();                                              \
    if (_e != hipSuccess)                                                           \
      return ::vh::set_error(VH_ERR_LAUNCH, "kernel launch failed: %s",            \
                             hipGetErrorString(_e));                                \
  } while (0)
