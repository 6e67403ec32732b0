// tpo_common.hpp -- shared device/host helpers for libtpo_hip (gfx950).
//
// Arithmetic contract (all kernels):
//   * Built with -ffp-contract=off: the only fused multiply-adds are the
//     explicit __builtin_fma calls below, which restate the order the
//     reference's nvcc build (default -fmad=true) contracts its distance sums
//     into:  x*x + y*y + z*z        -> fma(z,z, fma(x,x, y*y))
//            dist += diff*diff (KNN) -> fma(dk,dk, ... fma(d1,d1, d0*d0))
//   * float16 follows c10::Half: every + - * is computed and rounded to
//     binary16 on its own (native v_*_f16 ops; rounding a binary32 result to
//     binary16 equals one direct rounding since 24 >= 2*11+2), comparisons
//     are done on the exact values.
//   * Denormals are kept (-fno-gpu-flush-denormals-to-zero).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tpo.h"

namespace tpo {

typedef _Float16 half_t;

// ---------------------------------------------------------------- dtype traits
template <typename T> struct Lim;
template <> struct Lim<float> {
  __device__ static constexpr float inf() { return __builtin_inff(); }
};
template <> struct Lim<double> {
  __device__ static constexpr double inf() { return __builtin_inf(); }
};
template <> struct Lim<half_t> {
  __device__ static half_t inf() { return (half_t)__builtin_inff(); }
};

// Squared distance of chamfer.cu:64-67 / fps.cu:145 for the component
// differences (x, y, z).
__device__ __forceinline__ float sq3(float x, float y, float z) {
  return __builtin_fmaf(z, z, __builtin_fmaf(x, x, y * y));
}
__device__ __forceinline__ double sq3(double x, double y, double z) {
  return __builtin_fma(z, z, __builtin_fma(x, x, y * y));
}
__device__ __forceinline__ half_t sq3(half_t x, half_t y, half_t z) {
  return (half_t)((half_t)(x * x) + (half_t)(y * y)) + (half_t)(z * z);
}

// One step of the KNN distance accumulation (knn.cu:148-158, norm 2):
// first term diff*diff, later terms fma(diff, diff, acc); f16 rounds each op.
__device__ __forceinline__ float knn_acc2(float acc, float d, bool first) {
  return first ? d * d : __builtin_fmaf(d, d, acc);
}
__device__ __forceinline__ double knn_acc2(double acc, double d, bool first) {
  return first ? d * d : __builtin_fma(d, d, acc);
}
__device__ __forceinline__ half_t knn_acc2(half_t acc, half_t d, bool first) {
  half_t s = d * d;
  return first ? s : (half_t)(acc + s);
}
// norm 1 (knn.cu:154-156): dist += (diff > 0) ? diff : -diff
template <typename T>
__device__ __forceinline__ T knn_acc1(T acc, T d, bool first) {
  T a = d > (T)0 ? d : (T)(-d);
  // the sum starts at +0 (knn.cu:149): for d = +0 the first term is
  // 0 + (-0) = +0, so equal points are at +0, never -0
  return first ? (T)((T)0 + a) : (T)(acc + a);
}

// ------------------------------------------------------------ launch helpers
// Workgroups are dispatched round-robin over the 8 XCDs of MI355X.  Renumber
// so that consecutive logical blocks land on one XCD (and share its L2) when
// the grid divides evenly; otherwise keep the hardware order.
__device__ __forceinline__ int xcd_logical_block(int p, int grid) {
  if ((grid & 7) != 0) return p;
  return (p & 7) * (grid >> 3) + (p >> 3);
}

// Batch-affine block order: with B a multiple of 8 and `per` blocks per
// batch (grid = B * per), block p runs batch (p % 8) + 8 ((p / 8) / per),
// block (p / 8) % per of it.  Workgroups go to the XCDs round-robin by p, so
// every kernel that uses this order runs batch b on XCD b % 8: what one
// kernel writes for a batch is in that XCD's L2 when the next reads it.
// Returns false (and leaves b, j alone) when B is not a multiple of 8.
__device__ __forceinline__ bool batch_home_block(int p, int B, int per, int& b, int& j) {
  if ((B & 7) != 0) return false;
  const int s = p >> 3;
  b = __builtin_amdgcn_readfirstlane((p & 7) + 8 * (s / per));
  j = __builtin_amdgcn_readfirstlane(s % per);
  return true;
}

// readfirstlane makes the wave index provably wave-uniform, so values derived
// from it live in SGPRs and loads addressed by it become scalar loads.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// --------------------------------------------------------- atomics (no CAS)
__device__ __forceinline__ void atomic_add(float* p, float v) {
  (void)__hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void atomic_add(double* p, double v) {
  (void)__hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// binary16: packed add on the aligned 32-bit word with 0 in the other half,
// the same per-add rounding as the reference's __half2 atomics.
__device__ __forceinline__ void atomic_add(half_t* p, half_t v) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  uintptr_t a = (uintptr_t)p;
  h2* w = (h2*)(a & ~(uintptr_t)3);
  h2 val = (a & 2) ? h2{(half_t)0, v} : h2{v, (half_t)0};
  (void)__builtin_amdgcn_global_atomic_fadd_v2f16((__attribute__((address_space(1))) h2*)w, val);
}

// Index of cell (x, y, z) of a 16^3 grid along a 3-D Hilbert curve, by
// Skilling's transpose method ("Programming the Hilbert curve", AIP Conf.
// Proc. 707, 2004): undo the excess work from the top bit down, Gray-encode,
// then interleave the bits (x first) from the top.  Consecutive indices are
// neighbouring cells, so a run of points in this order is one compact region
// (a Morton run can jump between distant cells at an octant border).
__device__ __forceinline__ uint32_t hilbert3_16(uint32_t x, uint32_t y, uint32_t z) {
  uint32_t X[3] = {x, y, z};
#pragma unroll
  for (uint32_t Q = 8; Q > 1; Q >>= 1) {
    const uint32_t P = Q - 1;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (X[i] & Q) {
        X[0] ^= P;
      } else {
        const uint32_t t = (X[0] ^ X[i]) & P;
        X[0] ^= t;
        X[i] ^= t;
      }
    }
  }
  X[1] ^= X[0];
  X[2] ^= X[1];
  uint32_t t = 0;
#pragma unroll
  for (uint32_t Q = 8; Q > 1; Q >>= 1)
    if (X[2] & Q) t ^= Q - 1;
  uint32_t h = 0;
#pragma unroll
  for (int b = 3; b >= 0; --b)
#pragma unroll
    for (int i = 0; i < 3; ++i) h = (h << 1) | (((X[i] ^ t) >> b) & 1u);
  return h;
}

}  // namespace tpo

// ------------------------------------------------------------ host helpers
namespace tpo {
// Record an error message for tpo_last_error() and return the code.
int set_error(int code, const char* fmt, ...);
// After a launch: map hipGetLastError to TPO_ERR_LAUNCH.
int check_launch(const char* what);
}  // namespace tpo
