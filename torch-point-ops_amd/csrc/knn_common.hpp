// knn_common.hpp -- MinK pieces shared by the KNN forward kernels (knn.hip,
// knn_grid.hip): the reference's distance accumulation, its first-maximum
// slot rule, candidate masks, a register select tree and the row sort of
// knn_points(return_sorted=True).
#pragma once

#include "tpo_common.hpp"

#pragma clang fp contract(off)

namespace tpo {

constexpr int KNN_CHUNK = 32;

// Distance between the lane's query and reference r (knn.cu:148-158).
// DT > 0: compile-time dimension, query in registers; DT == 0: runtime D,
// query read through qp.
template <typename T, int DT, int NORM>
__device__ __forceinline__ T knn_dist(const T* qr, const T* __restrict__ qp,
                                      const T* __restrict__ r, int D) {
  T acc = (T)0;
  if constexpr (DT > 0) {
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      const T diff = (T)(qr[d] - r[d]);
      acc = NORM == 2 ? knn_acc2(acc, diff, d == 0) : knn_acc1(acc, diff, d == 0);
    }
  } else {
    for (int d = 0; d < D; ++d) {
      const T diff = (T)(qp[d] - r[d]);
      acc = NORM == 2 ? knn_acc2(acc, diff, d == 0) : knn_acc1(acc, diff, d == 0);
    }
  }
  return acc;
}

// First slot holding the maximum among slots [0, K) (mink.cuh:96-104).
template <typename T, int KC>
__device__ __forceinline__ void first_max(const T (&sd)[KC], int K, T& m, int& ms) {
  m = sd[0];
  ms = 0;
#pragma unroll
  for (int s = 1; s < KC; ++s) {
    if (s < K && sd[s] > m) {
      m = sd[s];
      ms = s;
    }
  }
}

// Broadcast a wave-uniform value into a VGPR so the subtractions that use it
// are VGPR-only VALU ops (an SGPR source costs 4 cycles per wave64 op).  The
// empty asm only pins the value to a VGPR: the compiler emits the move (and
// any wait it needs) itself.
__device__ __forceinline__ float to_vgpr(float s) {
  float v = s;
  asm("" : "+v"(v));
  return v;
}
__device__ __forceinline__ double to_vgpr(double s) { return s; }
__device__ __forceinline__ half_t to_vgpr(half_t s) { return s; }

// Inline asm on this GPU (gfx950, as gfx942) must not read an SGPR or vcc
// that a VALU op wrote fewer than two wait states before: the compiler
// inserts those waits between its own instructions but not inside or in
// front of an asm statement.  The asm below either reads VGPRs only or
// spaces each such read itself.  Likewise the compiler waits for an MFMA's
// result only before its own instructions: asm reading MFMA accumulators
// must follow (by a data dependence) a compiler-visible read of them.

// mask = 16 * mask + 8 (d0 < thr) + 4 (d1 < thr) + 2 (d2 < thr) + (d3 < thr):
// four compares into four SGPR pairs, then four add-with-carry doublings;
// each carry-in is read three instructions after its compare wrote it.
__device__ __forceinline__ uint32_t push_lt4(uint32_t mask, float d0, float d1, float d2, float d3,
                                             float thr) {
  uint32_t r;
  uint64_t c0, c1, c2, c3;
  asm("v_cmp_lt_f32 %1, %6, %10\n\t"
      "v_cmp_lt_f32 %2, %7, %10\n\t"
      "v_cmp_lt_f32 %3, %8, %10\n\t"
      "v_cmp_lt_f32 %4, %9, %10\n\t"
      "v_addc_co_u32 %0, vcc, %5, %5, %1\n\t"
      "v_addc_co_u32 %0, vcc, %0, %0, %2\n\t"
      "v_addc_co_u32 %0, vcc, %0, %0, %3\n\t"
      "v_addc_co_u32 %0, vcc, %0, %0, %4"
      : "=&v"(r), "=&s"(c0), "=&s"(c1), "=&s"(c2), "=&s"(c3)
      : "v"(mask), "v"(d0), "v"(d1), "v"(d2), "v"(d3), "v"(thr)
      : "vcc");
  return r;
}
template <typename T>
__device__ __forceinline__ uint32_t push_lt4(uint32_t mask, T d0, T d1, T d2, T d3, T thr) {
  return 16 * mask + 8 * (uint32_t)(d0 < thr) + 4 * (uint32_t)(d1 < thr) +
         2 * (uint32_t)(d2 < thr) + (uint32_t)(d3 < thr);
}

// Per-lane selects by a lane mask held in a VGPR (all ones: b, zero: a).
// v_bfi_b32 reads VGPRs only.  Kept as asm so that the compiler cannot turn
// the select trees below back into dynamically indexed (stack) arrays.
__device__ __forceinline__ uint32_t vsel_u32(uint32_t sel, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(sel), "v"(b), "v"(a));
  return r;
}
__device__ __forceinline__ float csel(uint32_t sel, float a, float b) {
  return __uint_as_float(vsel_u32(sel, __float_as_uint(a), __float_as_uint(b)));
}
__device__ __forceinline__ double csel(uint32_t sel, double a, double b) {
  const uint64_t x = __double_as_longlong(a), y = __double_as_longlong(b);
  const uint64_t lo = vsel_u32(sel, (uint32_t)x, (uint32_t)y);
  const uint64_t hi = vsel_u32(sel, (uint32_t)(x >> 32), (uint32_t)(y >> 32));
  return __longlong_as_double((long long)((hi << 32) | lo));
}
__device__ __forceinline__ half_t csel(uint32_t sel, half_t a, half_t b) {
  const uint32_t x = __builtin_bit_cast(uint16_t, a), y = __builtin_bit_cast(uint16_t, b);
  return __builtin_bit_cast(half_t, (uint16_t)vsel_u32(sel, x, y));
}
// all ones where bit k of x is set (one bit-field extract)
__device__ __forceinline__ uint32_t bit_mask(uint32_t x, int k) {
  return (uint32_t)((int32_t)(x << (31 - k)) >> 31);
}

// Slot ms of the lane's MinK takes (d, j): a mask and a select per slot,
// written with explicit selects so that the compiler cannot lower the
// dynamically indexed store into a branch tree (which lanes that diverge
// would all walk).
template <typename T, int KC>
__device__ __forceinline__ void mink_put(T (&sd)[KC], int (&si)[KC], int ms, T d, int j) {
  static_assert(KC <= 32, "one bit per slot");
  const uint32_t one = 1u << ms;
#pragma unroll
  for (int s = 0; s < KC; ++s) {
    const uint32_t hit = bit_mask(one, s);
    sd[s] = csel(hit, sd[s], d);
    si[s] = (int)vsel_u32(hit, (uint32_t)si[s], (uint32_t)j);
  }
}
template <typename T, int KC>
__device__ __forceinline__ void mink_put(T (&sd)[KC], int ms, T d) {
  static_assert(KC <= 32, "one bit per slot");
  const uint32_t one = 1u << ms;
#pragma unroll
  for (int s = 0; s < KC; ++s) sd[s] = csel(bit_mask(one, s), sd[s], d);
}

// d[c] for a per-lane c in [0, 32): a 5-level select tree over registers
// (a lane mask per level, 31 selects).
template <typename T>
__device__ __forceinline__ T select32(const T (&d)[KNN_CHUNK], int c) {
  T a[16], b[8], e[4], f[2];
  const uint32_t m0 = bit_mask(c, 0), m1 = bit_mask(c, 1), m2 = bit_mask(c, 2);
  const uint32_t m3 = bit_mask(c, 3), m4 = bit_mask(c, 4);
#pragma unroll
  for (int i = 0; i < 16; ++i) a[i] = csel(m0, d[2 * i], d[2 * i + 1]);
#pragma unroll
  for (int i = 0; i < 8; ++i) b[i] = csel(m1, a[2 * i], a[2 * i + 1]);
#pragma unroll
  for (int i = 0; i < 4; ++i) e[i] = csel(m2, b[2 * i], b[2 * i + 1]);
#pragma unroll
  for (int i = 0; i < 2; ++i) f[i] = csel(m3, e[2 * i], e[2 * i + 1]);
  return csel(m4, f[0], f[1]);
}

// knn_points(return_sorted=True) sorts each row with torch's sort along the
// last dim (knn/__init__.py:111-131).  For rows of at most 32 entries torch
// runs a 32-wide bitonic network (entries past the row invalid, sorting last)
// whose compare-exchange swaps unless the first key is valid and strictly
// less (NaN counts as largest) -- so ties come out in the network's order, not
// a stable one.  This replays that network on a lane's row in registers.
// Only the first KC positions can hold valid entries: KC is a power of two,
// every exchange within blocks of at most KC positions stays inside one
// block, and an exchange across position KC (a valid entry against an
// invalid one) runs in ascending direction, which never moves the entry up.
template <typename T>
__device__ __forceinline__ bool knn_isnan(T x) {
  return x != x;
}
template <typename T, int KC>
__device__ __forceinline__ void knn_sort_row(T (&d)[KC], int (&ix)[KC], uint32_t valid) {
  auto cas = [&](int a, int b, bool up) {  // branch-free compare-exchange
    const bool va = (valid >> a) & 1u, vb = (valid >> b) & 1u;
    const bool lt = !knn_isnan(d[a]) && (knn_isnan(d[b]) || d[a] < d[b]);
    const bool x = ((lt && va) || !vb) == up;
    const T da = d[a], db = d[b];
    const int ia = ix[a], ib = ix[b];
    d[a] = x ? db : da;
    d[b] = x ? da : db;
    ix[a] = x ? ib : ia;
    ix[b] = x ? ia : ib;
    valid ^= (x && va != vb) ? (1u << a) | (1u << b) : 0u;
  };
#pragma unroll
  for (int size = 2; size < 32; size *= 2)
#pragma unroll
    for (int stride = size / 2; stride > 0; stride /= 2)
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int a = 2 * t - (t & (stride - 1));
        if (a + stride < KC) cas(a, a + stride, (t & (size / 2)) != 0);
      }
#pragma unroll
  for (int stride = 16; stride > 0; stride /= 2)
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int a = 2 * t - (t & (stride - 1));
      if (a + stride < KC) cas(a, a + stride, false);
    }
}

// lane L of each 16-lane row, broadcast over the row (gfx950 DPP row_newbcast).
// Every lane reads a lane of its own row, so no old value is needed: without
// one the move folds into the VALU op that uses it whatever the schedule.
template <int L>
__device__ __forceinline__ float row_bcast(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x150 + L, 0xF,
                                                            0xF, true));
}
}  // namespace tpo
