// chamfer_common.hpp -- pieces shared by the chamfer forward kernels.  Every
// NaN / finiteness decision here is a test on the bit pattern, so it holds
// whatever floating-point assumptions a translation unit is compiled with.
#pragma once
#include "tpo_common.hpp"

namespace tpo {

constexpr int CH_WAVES = 4;  // waves per workgroup; they split the reference cloud
constexpr int CH_TILE = 16;  // references per tile of the tile-minimum argmin

constexpr uint32_t CH_BIG = 0x5d800000u;  // float bits of 2^60

__device__ __forceinline__ uint32_t abs_bits(float x) { return __float_as_uint(x) & 0x7fffffffu; }

__device__ __forceinline__ bool is_nan(float x) { return abs_bits(x) > 0x7f800000u; }
__device__ __forceinline__ bool is_nan(double x) {
  return ((uint64_t)__double_as_longlong(x) & 0x7fffffffffffffffull) > 0x7ff0000000000000ull;
}
__device__ __forceinline__ bool is_nan(half_t x) {
  return (__builtin_bit_cast(uint16_t, x) & 0x7fffu) > 0x7c00u;
}
__device__ __forceinline__ bool is_finite(float x) { return abs_bits(x) < 0x7f800000u; }
__device__ __forceinline__ bool is_finite(double x) {
  return ((uint64_t)__double_as_longlong(x) & 0x7fffffffffffffffull) < 0x7ff0000000000000ull;
}
__device__ __forceinline__ bool is_finite(half_t x) {
  return (__builtin_bit_cast(uint16_t, x) & 0x7fffu) < 0x7c00u;
}

template <typename T>
__device__ __forceinline__ bool finite3(const T* __restrict__ p) {
  return is_finite(p[0]) && is_finite(p[1]) && is_finite(p[2]);
}

// Squared distance with the reference's formula (chamfer.cu:64-67).
template <typename T>
__device__ __forceinline__ T ref_d(T qx, T qy, T qz, const T* __restrict__ r) {
  return sq3((T)(r[0] - qx), (T)(r[1] - qy), (T)(r[2] - qz));
}

// The wave's sum in lane 63 (the other lanes hold partial sums), in a fixed
// order by DPP adds: pairs, quads, 8 (half-row mirror), 16 (row mirror), then
// rows 0+1 and 2+3 (row_bcast:15) and all four (row_bcast:31).  double: the
// same sum by lane swaps, in every lane.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float ch_dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWMASK, 0xf, false));
}
__device__ __forceinline__ float wave_add63(float v) {
  v = ch_dpp_add<0xB1, 0xf>(v);
  v = ch_dpp_add<0x4E, 0xf>(v);
  v = ch_dpp_add<0x141, 0xf>(v);
  v = ch_dpp_add<0x140, 0xf>(v);
  v = ch_dpp_add<0x142, 0xa>(v);
  v = ch_dpp_add<0x143, 0xc>(v);
  return v;
}
__device__ __forceinline__ double wave_add63(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Wave minima of NaN-free values.
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ double wave_min(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmin(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ half_t wave_min(half_t v) { return (half_t)wave_min((float)v); }
__device__ __forceinline__ int wave_imin(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
  return v;
}

// The reference's result for one query over the references [c0, c1),
// computed by the whole wave (lanes stride the references).  chamfer.cu:55-82
// takes the first element of each 512-reference stage unconditionally and
// later ones on strict less; a stage replaces the stored result only when
// that is strictly greater (:159-162).  With finite distances this is the
// first index of the minimum.  With NaN distances: reference j counts only
// if neither D(j) nor D(512*floor(j/512)) is NaN, and a NaN D(0) makes the
// answer (NaN, 0).  Returns the minimum and first index over the counted
// references of the range ((+inf, INT_MAX) when none counts), or (NaN, 0).
template <typename T>
__device__ void chunk_scan(T qx, T qy, T qz, const T* __restrict__ rp, int c0, int c1, int lane,
                           T& out_d, int& out_i) {
  T d_ = Lim<T>::inf();
  int i_ = 0x7fffffff;
  for (int j = c0 + lane; j < c1; j += 64) {
    const T d = ref_d(qx, qy, qz, rp + 3 * j);
    const int h = j & ~511;
    const T dh = h == j ? d : ref_d(qx, qy, qz, rp + 3 * h);
    if (!is_nan(d) && !is_nan(dh) && (d < d_ || (d == d_ && i_ == 0x7fffffff))) {
      d_ = d;
      i_ = j;
    }
  }
  T md = wave_min(d_);
  int mi = wave_imin(d_ == md ? i_ : 0x7fffffff);
  if (c0 == 0) {
    const T d0 = ref_d(qx, qy, qz, rp);
    if (is_nan(d0)) {
      md = d0;
      mi = 0;
    }
  }
  out_d = md;
  out_i = mi;
}

// Final merge of the CH_WAVES chunk results of one query, in chunk (index)
// order with strict less, so ties keep the earlier chunk; a NaN result of the
// first chunk (chunk_scan's NaN rule) stands.  An index of INT_MAX from every
// chunk means an empty reference cloud: (0, 0) as the reference's zeroed
// outputs (chamfer.cu:176-181).
template <typename T, int STRIDE>
__device__ __forceinline__ void merge_chunks(const T* sd, const int* si, T& d, int& ix) {
  d = sd[0];
  ix = si[0];
#pragma unroll
  for (int v = 1; v < CH_WAVES; ++v) {
    const T dv = sd[v * STRIDE];
    if (!is_nan(d) && dv < d) {
      d = dv;
      ix = si[v * STRIDE];
    }
  }
  if (ix == 0x7fffffff) {
    d = (T)0;
    ix = 0;
  }
}

// Exact grid-search forward for float and half clouds (chamfer_grid.hip).
constexpr int CH_PRUNE_MIN = 2048;  // both clouds at least this large
int64_t chamfer_prune_workspace(int64_t B, int64_t N, int64_t M);
// dtype: TPO_F32 or TPO_F16.  `zero` (optional): a device word the sort
// kernel sets to 0 before the search runs (the loss reduction's counter).
void launch_chamfer_fwd_prune(int dtype, const void* x1, const void* x2, int B, int N, int M,
                              void* d1, void* d2, int32_t* i1, int32_t* i2, void* ws,
                              hipStream_t s, uint32_t* zero = nullptr);
void launch_chamfer_prune_stats(const void* ws, int64_t B, int64_t N, int64_t M, int64_t* out,
                                hipStream_t s);

}  // namespace tpo
