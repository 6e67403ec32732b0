// emd.hip -- earth mover's distance (approximate matching) for gfx950.
//
// Replaces approxmatch, matchcost, matchcostgrad1 and matchcostgrad2
// (emd.cu:18-303).  The algorithm is the reference's: mass multiL on every
// xyz1 point and multiR on every xyz2 point (emd.cu:21-28), then ten levels
// j = 7 .. -2 with level = -4^j (0 for the last, emd.cu:39-43), each of
// three passes over all n*m pairs with e(k,l) = exp(level * |p2_l - p1_k|^2)
// (the argument clamped to [-20, 20] for float16, emd.cu:77-80):
//   pass 1  ratioL[k] = remainL[k] / (1e-9 + sum_l e * remainR[l] + 1e-9)
//   pass 2  sumr = remainR[l] * sum_k e * ratioL[k];
//           ratioR[l] = min(remainR[l] / (sumr + 1e-9), 1) * remainR[l];
//           remainR[l] = max(0, remainR[l] - sumr)
//   pass 3  w = e * ratioL[k] * ratioR[l];  match[l][k] += w;
//           remainL[k] = max(0, remainL[k] - sum_l w)
// (1e-4 instead of 1e-9 for float16), then cost = sum d(k,l) * match[l][k].
// Arithmetic is at::opmath_type (float for float and half, double for
// double); remain/ratio/match values are rounded to the storage dtype as the
// reference stores them, and the reference's fminf/fmaxf narrow a double
// argument to float (emd.cu:134,136,178), which is kept.
//
// Design for MI355X (the reference runs one 512-thread block per cloud):
//   * each pass is a grid-wide sweep: a 512-thread workgroup owns 64 points
//     (one per lane) and its eight waves each sum over an eighth of the other
//     cloud, staged through LDS, combined in fixed order;
//   * exponentials that are +0 in all 64 lanes (arguments below the float
//     or double underflow, the steep levels on distant points) are skipped
//     with a wave-uniform branch, which changes no sum; each cloud's points
//     are listed as k-d tree leaves (Morton cells above 4096 points) so a
//     wave's 64 points are neighbours, and at the steep levels the points of
//     the other cloud beyond reach of the wave's box are left out altogether;
//     flat levels drop the zero tests once they stop paying;
//   * the float paths' exp is a two-term Cody-Waite reduction on the
//     hardware exp2 (at most 1.24 ulp from exp over [-87, 0], measured);
//     their last level's exp(0 * d) is 0 * d + 1 exactly;
//   * pass 3 of level j and pass 1 of level j-1 need the same inputs, so they
//     share one sweep (two exponentials per pair): 21 dependent sweeps;
//     levels j and j-1 differ by a factor 4, so in float32 both exponentials
//     share one argument reduction (4x splits exactly as 4h + 4l): one more
//     exp2 and fma give exp(4x) bit for bit;
//   * match is not accumulated in HBM level by level: the per-level ratioL
//     and ratioR are kept, and one final pass forms
//     match[l][k] = sum_j e_j(k,l) * ratioL_j[k] * ratioR_j[l] in level order
//     (each addition rounded as the reference's +=), writes it once and fuses
//     matchcost's sum of d * match into the same pass;
//   * the backward reads match once: a tile's column sums (grad_xyz1) stay
//     in registers and its row sums (grad_xyz2) are reduced across the wave;
//   * every sum has a fixed order, so results are deterministic.
// The summation orders differ from the reference's sequential loops and the
// exponential is ROCm's, so parity is to a tolerance, not bit-exact.
#include "tpo_common.hpp"

#include <algorithm>
#include <type_traits>

namespace tpo {
namespace {

constexpr int EMD_LEVELS = 10;       // j = 7 .. -2
constexpr int EMD_THREADS = 256;     // 4 waves
constexpr int EMD_SWEEP_THREADS = 512;  // 8 waves per 64 points of a sweep
constexpr int EMD_MATCH_ROWS = 32;   // match rows per workgroup of the final pass
constexpr int EMD_G1_ROWS = 128;     // match rows per grad_xyz1 partial

template <typename T> struct EmdV { typedef float type; };
template <> struct EmdV<double> { typedef double type; };

// level of step t = 7 - j (emd.cu:40-43)
template <typename V>
__device__ __forceinline__ V emd_level(int t) {
  return t < 8 ? -(V)(1 << (14 - 2 * t)) : (t == 8 ? (V)-0.25 : (V)0);
}
// epsilon of emd.cu:55,89,133: static_cast<opmath_t>(1e-9f), 1e-4f for half
template <typename T, typename V>
__device__ __forceinline__ V emd_eps() {
  return std::is_same<T, half_t>::value ? (V)1e-4f : (V)1e-9f;
}
// an opmath value stored as scalar_t and read back
template <typename T, typename V>
__device__ __forceinline__ V emd_st(V v) {
  if constexpr (std::is_same<T, half_t>::value) return (V)(half_t)v;
  return v;
}
// exp(x) of the float paths (x <= 0 here, or NaN): 2^(x log2 e) with
// x log2 e split as h + l by Cody and Waite's two-term reduction,
// h = fl(x L1), l = fma(x, L2, fma(x, L1, -h)) where L1 + L2 = log2 e to 48
// bits; 2^h from the hardware exp2 (v_exp_f32) and 2^l = 1 + l ln2 to within
// (l ln2)^2 / 2 < 2^-33 since |l| < 2^-16.  Arguments below -150 give +0
// (the value is below 2^-216); NaN stays NaN.  Results below 2^-126 may
// flush to 0, far below every term these sums can resolve.
__device__ __forceinline__ float emd_exp(float x) {
  x = x < -150.f ? -150.f : x;
  constexpr float L1 = 1.44269502162933349609375f;  // fl(log2 e)
  constexpr float L2 = 1.925962989e-8f;             // log2 e - L1
  const float h = x * L1;
  const float l = __builtin_fmaf(x, L2, __builtin_fmaf(x, L1, -h));
  const float r = __builtin_amdgcn_exp2f(h);
  return __builtin_fmaf(r, l * 0.693147180559945309f, r);
}
__device__ __forceinline__ double emd_exp(double x) { return exp(x); }
// emd_exp(x) and emd_exp(4x) from one reduction: scaling by 4 is exact, so
// 4x splits as 4h + 4l and the second value takes one more exp2 and fma, bit
// for bit what emd_exp(4x) returns (for 4x below -150, where that clamps,
// exp2(4h) is +0 as well).
__device__ __forceinline__ void emd_exp_x4(float x, float& e1, float& e4) {
  x = x < -150.f ? -150.f : x;
  constexpr float L1 = 1.44269502162933349609375f;
  constexpr float L2 = 1.925962989e-8f;
  const float h = x * L1;
  const float l = __builtin_fmaf(x, L2, __builtin_fmaf(x, L1, -h));
  const float t = l * 0.693147180559945309f;
  const float r = __builtin_amdgcn_exp2f(h);
  const float r4 = __builtin_amdgcn_exp2f(4.f * h);
  e1 = __builtin_fmaf(r, t, r);
  e4 = __builtin_fmaf(r4, 4.f * t, r4);
}
template <typename T, typename V>
__device__ __forceinline__ V emd_e(V level, V d) {
  // the last level: exp(0 * d) = 1 for finite d, NaN otherwise, = 0 * d + 1
  // (float paths; the double kernels keep their registers for exp)
  if constexpr (!std::is_same<V, double>::value)
    if (level == (V)0) return level * d + (V)1;
  V a = level * d;
  if constexpr (std::is_same<T, half_t>::value)
    a = a < (V)-20 ? (V)-20 : (a > (V)20 ? (V)20 : a);
  return emd_exp(a);
}
// Below these arguments exp() is exactly +0 (float: e^-103.98 is half the
// smallest denormal; double: e^-745.2), so a term e * w adds exactly nothing
// to a sum of non-negative terms; float16 clamps its argument at -20.
template <typename T, typename V>
__device__ __forceinline__ V emd_zero_below() {
  return std::is_same<T, double>::value ? (V)-760 : (V)-120;
}
// A distance above this makes exp(level * d) exactly +0 (level < 0):
// level * d is then below zb within a few ulps, far inside the margin between
// zb and the underflow point; never for level 0.  Testing d against it saves
// the product level * d.
template <typename T, typename V>
__device__ __forceinline__ V emd_zero_dist(V level) {
  return level < (V)0 ? emd_zero_below<T, V>() / level : (V)__builtin_inf();
}
// True when exp(level * d) is +0 in every lane of the wave, so the wave can
// skip the exponential and its products (wave-uniform branch).  A NaN
// distance is never "above", so NaN still propagates.
template <typename T, typename V>
__device__ __forceinline__ bool emd_wave_zero(V level, V d) {
  if constexpr (std::is_same<T, half_t>::value) return false;
  return __builtin_amdgcn_ballot_w64(!(d > emd_zero_dist<T, V>(level))) == 0;
}
// fminf(x, 1.0f) / fmaxf(0.0f, x) of emd.cu:134,136,178 (float functions)
template <typename V>
__device__ __forceinline__ V emd_min1(V a) { return (V)fminf((float)a, 1.0f); }
template <typename V>
__device__ __forceinline__ V emd_max0(V a) { return (V)fmaxf(0.0f, (float)a); }
__device__ __forceinline__ float emd_fma(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double emd_fma(double a, double b, double c) { return __builtin_fma(a, b, c); }

template <typename V>
__device__ __forceinline__ V wave_sum(V v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// The wave's sum in lane 63 (float; the other lanes hold partial sums), by
// DPP adds in a fixed order: pairs, quads, 8 (half-row mirror), 16 (row
// mirror), then rows 0+1 and 2+3 (row_bcast:15) and all four (row_bcast:31).
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWMASK, 0xf, false));
}
__device__ __forceinline__ float wave_total63(float v) {
  v = dpp_add<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141, 0xf>(v);  // row_half_mirror
  v = dpp_add<0x140, 0xf>(v);  // row_mirror
  v = dpp_add<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
  v = dpp_add<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
  return v;
}
__device__ __forceinline__ double wave_total63(double v) { return wave_sum(v); }
// Wave minimum / maximum in every lane (float: DPP into lane 63, whose value
// is read back; double: lane swaps).  The masked-off rows of a row_bcast step
// take the identity (+inf / -inf).
template <int CTRL, int ROWMASK, bool MAX>
__device__ __forceinline__ float dpp_minmax(float v) {
  const float id = MAX ? -__builtin_inff() : __builtin_inff();
  const float o = __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(id), __float_as_int(v), CTRL, ROWMASK, 0xf, false));
  return MAX ? fmaxf(v, o) : fminf(v, o);
}
template <bool MAX>
__device__ __forceinline__ float wave_minmax(float v) {
  v = dpp_minmax<0xB1, 0xf, MAX>(v);
  v = dpp_minmax<0x4E, 0xf, MAX>(v);
  v = dpp_minmax<0x141, 0xf, MAX>(v);
  v = dpp_minmax<0x140, 0xf, MAX>(v);
  v = dpp_minmax<0x142, 0xa, MAX>(v);
  v = dpp_minmax<0x143, 0xc, MAX>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
template <bool MAX>
__device__ __forceinline__ double wave_minmax(double v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const double u = __shfl_xor(v, o, 64);
    v = MAX ? fmax(v, u) : fmin(v, u);
  }
  return v;
}

// Workspace, array-major over the clouds (opmath values):
//   p1[B][n][4], p2[B][m][4]   coordinates (x, y, z, 0)
//   reml[B][n], remr[B][m]     remaining mass
//   rl[B][10][n], rr[B][10][m] ratioL / ratioR of every level
//   cost[B][gy][gx]            matchcost partials of the final pass
//   g1[B][nchunk][n][3]        grad_xyz1 partials of the backward (per row tile)
//   g2[B][gx][m][3]            grad_xyz2 partials of the backward (per column tile)
//   ord1[B][n], ord2[B][m]     int32: each cloud's points in sweep order
struct EmdLayout {
  int64_t p1, p2, reml, remr, rl, rr, cost, g1, g2, ord1, ord2, total;
  int gx, gy, nchunk;
};
template <typename V>
inline EmdLayout emd_layout(int64_t B, int64_t n, int64_t m) {
  EmdLayout L;
  L.gx = (int)((n + EMD_THREADS - 1) / EMD_THREADS);
  L.gy = (int)((m + EMD_MATCH_ROWS - 1) / EMD_MATCH_ROWS);
  L.nchunk = (int)((m + EMD_G1_ROWS - 1) / EMD_G1_ROWS);
  auto al = [](int64_t v) { return (v + 255) / 256 * 256; };
  const int64_t s = (int64_t)sizeof(V);
  int64_t o = 0;
  L.p1 = o; o += al(B * n * 4 * s);
  L.p2 = o; o += al(B * m * 4 * s);
  L.reml = o; o += al(B * n * s);
  L.remr = o; o += al(B * m * s);
  L.rl = o; o += al(B * EMD_LEVELS * n * s);
  L.rr = o; o += al(B * EMD_LEVELS * m * s);
  L.cost = o; o += al(B * (int64_t)L.gx * L.gy * s);
  L.g1 = o; o += al(B * (int64_t)L.nchunk * n * 3 * s);
  L.g2 = o; o += al(B * (int64_t)L.gx * m * 3 * s);
  L.ord1 = o; o += al(B * n * 4);
  L.ord2 = o; o += al(B * m * 4);
  L.total = o;
  return L;
}

// ---------------------------------------------------------------- forward

template <typename T>
__global__ __launch_bounds__(EMD_THREADS) void emd_prep_kernel(
    const T* __restrict__ xyz1, const T* __restrict__ xyz2, int n, int m, float mult_l,
    float mult_r, typename EmdV<T>::type* __restrict__ p1, typename EmdV<T>::type* __restrict__ p2,
    typename EmdV<T>::type* __restrict__ reml, typename EmdV<T>::type* __restrict__ remr) {
  typedef typename EmdV<T>::type V;
  const int64_t b = blockIdx.y;
  const int i = blockIdx.x * EMD_THREADS + threadIdx.x;
  if (i < n) {
    const T* s = xyz1 + (b * n + i) * 3;
    V* d = p1 + (b * n + i) * 4;
    d[0] = (V)s[0]; d[1] = (V)s[1]; d[2] = (V)s[2]; d[3] = (V)0;
    reml[b * n + i] = emd_st<T, V>((V)mult_l);
  }
  if (i < m) {
    const T* s = xyz2 + (b * m + i) * 3;
    V* d = p2 + (b * m + i) * 4;
    d[0] = (V)s[0]; d[1] = (V)s[1]; d[2] = (V)s[2]; d[3] = (V)0;
    remr[b * m + i] = emd_st<T, V>((V)mult_r);
  }
}

// The points of one cloud (blockIdx.y + first: 0 = xyz1, 1 = xyz2) listed so
// that every run of 64 (one sweep wave's own points) lies close together:
// the steep levels' exponentials then vanish in all of a wave's lanes at
// once, and far points of the other cloud drop out of the wave's sweep.
// Which wave a point sits in changes no result: its sums run over the other
// cloud in a fixed order and a skipped term is exactly zero.
// Clouds of more than EMD_KD_MAX points: the cell of a 16^3 grid over the
// bounding box, in Morton order of the cells (counting sort in LDS; the order
// inside a cell is whatever the atomics give).
constexpr int EMD_ORDER_THREADS = 1024;
constexpr int EMD_OGRID = 16;
constexpr int EMD_OCELLS = EMD_OGRID * EMD_OGRID * EMD_OGRID;

__device__ __forceinline__ uint32_t emd_spread3(uint32_t v) {  // 4 bits -> every third bit
  v &= 0xf;
  v = (v | (v << 4)) & 0x0c3;
  v = (v | (v << 2)) & 0x249;
  return v;
}

template <typename T>
__global__ __launch_bounds__(EMD_ORDER_THREADS) void emd_order_kernel(
    const T* __restrict__ xyz1, const T* __restrict__ xyz2, int n, int m, int* __restrict__ ord1,
    int* __restrict__ ord2, int first) {
  __shared__ uint32_t s_cnt[EMD_OCELLS];
  __shared__ float s_box[6][EMD_ORDER_THREADS / 64];
  __shared__ uint32_t s_part[EMD_ORDER_THREADS / 64];
  const int64_t b = blockIdx.x;
  const bool two = blockIdx.y + first != 0;
  const int N = two ? m : n;
  const T* P = two ? xyz2 + b * m * 3 : xyz1 + b * n * 3;
  int* ord = two ? ord2 + b * m : ord1 + b * n;
  const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
  float lo[3] = {__builtin_inff(), __builtin_inff(), __builtin_inff()};
  float hi[3] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
  for (int k = tid; k < N; k += EMD_ORDER_THREADS) {
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const float v = (float)P[3 * k + c];
      lo[c] = fminf(lo[c], v);
      hi[c] = fmaxf(hi[c], v);
    }
  }
#pragma unroll
  for (int c = 0; c < 3; ++c) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      lo[c] = fminf(lo[c], __shfl_xor(lo[c], o, 64));
      hi[c] = fmaxf(hi[c], __shfl_xor(hi[c], o, 64));
    }
    if (lane == 0) {
      s_box[c][w] = lo[c];
      s_box[3 + c][w] = hi[c];
    }
  }
  for (int c = tid; c < EMD_OCELLS; c += EMD_ORDER_THREADS) s_cnt[c] = 0;
  __syncthreads();
  float org[3], scl[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    float a = __builtin_inff(), z = -__builtin_inff();
    for (int v = 0; v < EMD_ORDER_THREADS / 64; ++v) {
      a = fminf(a, s_box[c][v]);
      z = fmaxf(z, s_box[3 + c][v]);
    }
    const float ext = z - a;
    org[c] = a;
    scl[c] = (ext > 0.f && ext < __builtin_inff()) ? (float)EMD_OGRID / ext : 0.f;
  }
  auto cell_of = [&](int k) -> uint32_t {
    uint32_t cc[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const float f = ((float)P[3 * k + c] - org[c]) * scl[c];
      int i = (f == f) ? (int)f : 0;  // NaN -> cell 0
      cc[c] = (uint32_t)(i < 0 ? 0 : (i > EMD_OGRID - 1 ? EMD_OGRID - 1 : i));
    }
    return emd_spread3(cc[0]) | (emd_spread3(cc[1]) << 1) | (emd_spread3(cc[2]) << 2);
  };
  for (int k = tid; k < N; k += EMD_ORDER_THREADS) atomicAdd(&s_cnt[cell_of(k)], 1u);
  __syncthreads();
  {  // exclusive scan of the counters, EMD_OCELLS / EMD_ORDER_THREADS per thread
    constexpr int PER = EMD_OCELLS / EMD_ORDER_THREADS;
    uint32_t v[PER], sum = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      v[i] = s_cnt[tid * PER + i];
      sum += v[i];
    }
    uint32_t incl = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t o = (uint32_t)__shfl_up((int)incl, d, 64);
      if (lane >= d) incl += o;
    }
    if (lane == 63) s_part[w] = incl;
    __syncthreads();
    uint32_t run = incl - sum;
    for (int v2 = 0; v2 < w; ++v2) run += s_part[v2];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      s_cnt[tid * PER + i] = run;
      run += v[i];
    }
  }
  __syncthreads();
  for (int k = tid; k < N; k += EMD_ORDER_THREADS) ord[atomicAdd(&s_cnt[cell_of(k)], 1u)] = k;
}

// Clouds of at most EMD_KD_MAX points: the leaves of a k-d tree whose leaves
// are the runs of 64 (the last one shorter).  A node of g runs splits into
// floor(g / 2) runs and the rest, across its longest extent, at the rank
// 64 floor(g / 2) along that axis.  Morton runs jump between distant cells at
// the octant borders, and a wave holding such a run reaches most of the
// other cloud; the tree's leaves are compact boxes.
//   Three arrays list the points ordered by x, y and z: keys are the
// coordinate quantised to 20 bits over the cloud's box, then the point (one
// 32-bit word), placed by a counting sort on the top EMD_KD_BBITS bits (the
// order inside a bin is whatever the atomics give: a split then errs by at
// most a bin, 1/512 of the box).  Each node is a segment of each array; its
// extents are read off its first and last keys, its split marks the points
// of the lower part along its axis, and a stable partition by that mark
// (prefix sums of the marks) orders its segment of the other two arrays the
// same way, so every node stays one segment in all three.  The x array's
// final order is the list.
constexpr int EMD_KD_MAX = 4096;
constexpr int EMD_KD_NODES = EMD_KD_MAX / 64;
constexpr int EMD_KD_QBITS = 20;
constexpr int EMD_KD_BBITS = 9;
constexpr int EMD_KD_BINS = 1 << EMD_KD_BBITS;

// inclusive prefix sum over the 64 lanes (all active): row_shr 1, 2, 4, 8
// within rows of 16 (lanes without a source read 0), then row_bcast:15 into
// rows 1, 3 and row_bcast:31 into rows 2, 3
template <int CTRL, int ROWMASK>
__device__ __forceinline__ int emd_dpp0(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWMASK, 0xf, true);
}
__device__ __forceinline__ int emd_wave_scan(int v) {
  v += emd_dpp0<0x111, 0xf>(v);
  v += emd_dpp0<0x112, 0xf>(v);
  v += emd_dpp0<0x114, 0xf>(v);
  v += emd_dpp0<0x118, 0xf>(v);
  v += emd_dpp0<0x142, 0xa>(v);
  v += emd_dpp0<0x143, 0xc>(v);
  return v;
}
// sum of the per-wave totals tot[0 .. w) (w = this wave; at most 64 waves)
__device__ __forceinline__ int emd_waves_before(const int* tot, int nw, int w) {
  const int lane = lane_id();
  const int t = lane < nw ? tot[lane] : 0;
  return __builtin_amdgcn_readlane(emd_wave_scan(t) - t, w);
}

template <typename T>
__global__ __launch_bounds__(EMD_ORDER_THREADS) void emd_kd_order_kernel(
    const T* __restrict__ xyz1, const T* __restrict__ xyz2, int n, int m, int* __restrict__ ord1,
    int* __restrict__ ord2, int first) {
  constexpr int TH = EMD_ORDER_THREADS, NWV = TH / 64;
  constexpr int PER = EMD_KD_MAX / TH;  // consecutive positions a thread (one run of 64)
  static_assert(EMD_KD_BINS <= TH, "one bin of each axis a thread");
  __shared__ __align__(16) uint32_t s_key[3][EMD_KD_MAX];
  __shared__ __align__(16) uint8_t s_flag[EMD_KD_MAX];
  __shared__ int s_cnt[3][EMD_KD_BINS];
  __shared__ float s_box[6][NWV];
  __shared__ int s_wsum[3][NWV];
  __shared__ int s_nstart[2][EMD_KD_NODES], s_ngrp[2][EMD_KD_NODES], s_nn[2];
  __shared__ int s_nlow[EMD_KD_NODES], s_naxis[EMD_KD_NODES], s_nbase[3][EMD_KD_NODES];
  __shared__ uint8_t s_nog[EMD_KD_NODES];  // node of each run of 64
  const int64_t b = blockIdx.x;
  const bool two = blockIdx.y + first != 0;
  const int N = two ? m : n;
  const T* P = two ? xyz2 + b * m * 3 : xyz1 + b * n * 3;
  int* ord = two ? ord2 + b * m : ord1 + b * n;
  const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
  if (N <= 0 || N > EMD_KD_MAX) return;
  const int i0 = tid * PER;  // this thread's positions i0 .. i0 + PER - 1
  // ---- this thread's points (positions = point indices here), the box ----
  float pc[PER][3];
  float lo[3] = {__builtin_inff(), __builtin_inff(), __builtin_inff()};
  float hi[3] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
#pragma unroll
  for (int u = 0; u < PER; ++u) {
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      pc[u][c] = i0 + u < N ? (float)P[3 * (i0 + u) + c] : 0.f;
      if (i0 + u < N) {
        lo[c] = fminf(lo[c], pc[u][c]);
        hi[c] = fmaxf(hi[c], pc[u][c]);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    lo[c] = wave_minmax<false>(lo[c]);
    hi[c] = wave_minmax<true>(hi[c]);
    if (lane == 0) {
      s_box[c][w] = lo[c];
      s_box[3 + c][w] = hi[c];
    }
  }
  if (tid < EMD_KD_BINS) {
#pragma unroll
    for (int c = 0; c < 3; ++c) s_cnt[c][tid] = 0;
  }
  __syncthreads();
  float scl[3], unit[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    float a = __builtin_inff(), z = -__builtin_inff();
    for (int v = 0; v < NWV; ++v) {
      a = fminf(a, s_box[c][v]);
      z = fmaxf(z, s_box[3 + c][v]);
    }
    const float ext = z - a;
    const bool ok = ext > 0.f && ext < __builtin_inff();
    lo[c] = a;
    scl[c] = ok ? (float)(1 << EMD_KD_QBITS) / ext : 0.f;
    unit[c] = ok ? ext / (float)(1 << EMD_KD_QBITS) : 0.f;
  }
  // ---- keys, and the three counting sorts at once ----
  uint32_t kv[3][PER];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const float f = (pc[u][c] - lo[c]) * scl[c];
      const float q = f == f ? fminf(fmaxf(f, 0.f), (float)((1 << EMD_KD_QBITS) - 1)) : 0.f;
      kv[c][u] = ((uint32_t)q << 12) | (uint32_t)(i0 + u);
      if (i0 + u < N) atomicAdd(&s_cnt[c][kv[c][u] >> (32 - EMD_KD_BBITS)], 1);
    }
  }
  __syncthreads();
  {  // exclusive prefix sums of the bins: thread t < EMD_KD_BINS holds bin t of each axis
    int v[3], incl[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      v[c] = tid < EMD_KD_BINS ? s_cnt[c][tid] : 0;
      incl[c] = emd_wave_scan(v[c]);
      if (lane == 63) s_wsum[c][w] = incl[c];
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const int off = incl[c] - v[c] + emd_waves_before(s_wsum[c], NWV, w);
      if (tid < EMD_KD_BINS) s_cnt[c][tid] = off;
    }
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < 3; ++c) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      if (i0 + u < N) s_key[c][atomicAdd(&s_cnt[c][kv[c][u] >> (32 - EMD_KD_BBITS)], 1)] = kv[c][u];
    }
  }
  // ---- the tree, a level at a time ----
  const int G = (N + 63) >> 6;  // runs of 64
  if (tid == 0) {
    s_nstart[0][0] = 0;
    s_ngrp[0][0] = G;
    s_nn[0] = 1;
  }
  __syncthreads();
  int cur = 0;
  for (int lev = 0; (1 << lev) < G; ++lev) {
    if (w == 0) {  // a lane per node: its axis and split, and the next level's nodes
      const int nn = s_nn[cur];
      int st = 0, g = 0, low = 0, ax = 0, nch = 0;
      if (lane < nn) {
        st = s_nstart[cur][lane];
        g = s_ngrp[cur][lane];
        nch = 1;
        if (g >= 2) {
          const int e = min(st + 64 * g, N) - 1;
          float best = -1.f;
#pragma unroll
          for (int c = 0; c < 3; ++c) {
            const int d = (int)(s_key[c][e] >> 12) - (int)(s_key[c][st] >> 12);
            const float ext = (float)(d < 0 ? -d : d) * unit[c];
            if (ext > best) {
              best = ext;
              ax = c;
            }
          }
          low = 64 * (g >> 1);
          nch = 2;
        }
      }
      const int incl = emd_wave_scan(nch);
      const int pos = incl - nch, nx = cur ^ 1;
      if (lane < nn) {
        s_nlow[lane] = low;
        s_naxis[lane] = ax;
        for (int q = 0; q < g; ++q) s_nog[(st >> 6) + q] = (uint8_t)lane;
        s_nstart[nx][pos] = st;
        s_ngrp[nx][pos] = nch == 2 ? g >> 1 : g;
        if (nch == 2) {
          s_nstart[nx][pos + 1] = st + low;
          s_ngrp[nx][pos + 1] = g - (g >> 1);
        }
      }
      if (lane == 63) s_nn[nx] = incl;
    }
    __syncthreads();
    // this thread's node (its PER positions lie in one run of 64)
    const bool act = i0 < N;
    const int nd = act ? s_nog[i0 >> 6] : 0;
    const int low = act ? s_nlow[nd] : 0, ax = s_naxis[nd], st = s_nstart[cur][nd];
    const bool split = low > 0;
    // mark the points of each node's lower part along its axis
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const uint4 q4 = act ? *reinterpret_cast<const uint4*>(&s_key[c][i0]) : make_uint4(0, 0, 0, 0);
      kv[c][0] = q4.x;
      kv[c][1] = q4.y;
      kv[c][2] = q4.z;
      kv[c][3] = q4.w;
    }
    if (split) {  // the axis array's keys again, read from LDS (no indexed registers)
      const uint4 q4 = *reinterpret_cast<const uint4*>(&s_key[ax][i0]);
      const uint32_t ka[PER] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
      for (int u = 0; u < PER; ++u)
        if (i0 + u < N) s_flag[ka[u] & 0xfff] = (uint8_t)(i0 + u - st < low);
    }
    __syncthreads();
    // stable partition of each splitting node's segment in the other two
    // arrays: prefix sums of the marks in array order, then every key to its
    // new position
    int f[3][PER], excl[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      int run = 0;
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        f[c][u] = i0 + u < N ? (int)s_flag[kv[c][u] & 0xfff] : 0;
        run += f[c][u];
      }
      const int incl = emd_wave_scan(run);
      if (lane == 63) s_wsum[c][w] = incl;
      excl[c] = incl - run;
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      excl[c] += emd_waves_before(s_wsum[c], NWV, w);
      if (act && i0 == st) s_nbase[c][nd] = excl[c];  // the node's first position
    }
    __syncthreads();
    if (split) {
#pragma unroll
      for (int c = 0; c < 3; ++c) {
        if (c == ax) continue;
        const int base = s_nbase[c][nd];
        int e = excl[c];
#pragma unroll
        for (int u = 0; u < PER; ++u) {
          const int i = i0 + u;
          if (i < N) {
            const int lb = e - base;  // marked points before i in the node
            s_key[c][f[c][u] ? st + lb : st + low + (i - st - lb)] = kv[c][u];
          }
          e += f[c][u];
        }
      }
    }
    __syncthreads();
    cur ^= 1;
  }
  for (int i = tid; i < N; i += TH) ord[i] = (int)(s_key[0][i] & 0xfff);
}

// One point of the coordinate arrays (x, y, z, unused), read whole.
template <typename V>
struct __attribute__((aligned(4 * sizeof(V)))) EmdPt {
  V x, y, z, w;
};

// Sums over the "other" cloud for one own point per lane (own: the lane's
// point is real; the sums of the other lanes are not used); the waves of the
// workgroup take an equal share of the other points each.  NS = 1 sums
// e(la)*wa; NS = 2 also sums e(lb)*wb with the same distances.  PR: leave
// out the points far from every own point of the wave (below).
template <typename T, int NS, bool PR>
__device__ __forceinline__ void emd_sweep(const typename EmdV<T>::type* __restrict__ other, int cnt,
                                          bool own, typename EmdV<T>::type x,
                                          typename EmdV<T>::type y, typename EmdV<T>::type z,
                                          typename EmdV<T>::type la,
                                          const typename EmdV<T>::type* __restrict__ wa,
                                          typename EmdV<T>::type lb,
                                          const typename EmdV<T>::type* __restrict__ wb,
                                          typename EmdV<T>::type* sums) {
  typedef typename EmdV<T>::type V;
  constexpr int NW = EMD_SWEEP_THREADS / 64;
  __shared__ V s_part[NS][NW - 1][64];
  const int w = wave_id(), lane = lane_id();
  const int q0 = (int)((int64_t)cnt * w / NW), q1 = (int)((int64_t)cnt * (w + 1) / NW);
  V sa = (V)0, sb = (V)0;
  // The wave stages its share of the other cloud 64 points at a time in its
  // own slice of LDS: lane i loads point i of the next chunk (vector loads,
  // issued before the current chunk is processed), then every lane reads the
  // chunk's points back as broadcasts.  The points are taken in batches of U;
  // one wave-uniform test per level decides whether any of the batch's
  // exponentials can be non-zero.  Terms are added in point order, as in a
  // plain loop.
  constexpr int C = 64, U = 8;
  __shared__ EmdPt<V> s_pt[NW][C];  // (x, y, z, wa)
  __shared__ V s_wb[NS == 2 ? NW : 1][C];
  const V ta = emd_zero_dist<T, V>(la), tb = emd_zero_dist<T, V>(lb);
  // float32, two levels a factor 4 apart (every fused sweep but the last):
  // both exponentials come from one argument reduction (emd_exp_x4).
  // float16 clamps each argument at -20, which breaks the scaling; float64
  // keeps its library exp.
  const bool pow4 = std::is_same<T, float>::value && NS == 2 && lb != (V)0 && la == (V)4 * lb;
  // Far points.  The wave's own points are neighbours in space (the sweep
  // takes them as k-d tree leaves), so many points of the other cloud lie
  // farther from the box of the wave's real own points than the zero
  // distance of every level summed here (with a relative margin of 2^-10, far
  // above the rounding of the box distance and of d): each of their terms is
  // exactly +0 in every real lane, and they are left out of the batches.  The
  // remaining points are summed in the same order, so the sums keep their
  // bits (for the finite weights these sweeps carry).  A wave with a
  // non-finite own coordinate leaves nothing out, nor does float16 (its
  // exponentials never vanish); a non-finite point of the other cloud is
  // always kept, so NaN still propagates.
  V reach = NS == 2 ? (ta > tb ? ta : tb) : ta;  // +inf for level 0
  if constexpr (std::is_same<T, half_t>::value) reach = (V)__builtin_inf();
  bool prune = false;
  V olo[3], ohi[3];
  if constexpr (PR) {
    const bool fin = __builtin_isfinite(x) && __builtin_isfinite(y) && __builtin_isfinite(z);
    if (__builtin_amdgcn_ballot_w64(own && !fin) != 0) reach = (V)__builtin_inf();
    prune = reach < (V)__builtin_inf();
  }
  if (prune) {
    const V inf = (V)__builtin_inf();
    olo[0] = wave_minmax<false>(own ? x : inf);
    olo[1] = wave_minmax<false>(own ? y : inf);
    olo[2] = wave_minmax<false>(own ? z : inf);
    ohi[0] = wave_minmax<true>(own ? x : -inf);
    ohi[1] = wave_minmax<true>(own ? y : -inf);
    ohi[2] = wave_minmax<true>(own ? z : -inf);
    reach *= (V)1 + (V)1 / (V)1024;
  }
  const EmdPt<V>* op = (const EmdPt<V>*)other;
  EmdPt<V> nr;
  V nb = (V)0;
  auto fetch = [&](int c0) {
    const int qq = c0 + lane;
    if (qq < q1) {
      const EmdPt<V> g = op[qq];
      nr = EmdPt<V>{g.x, g.y, g.z, wa[qq]};
      if constexpr (NS == 2) nb = wb[qq];
    } else {
      nr = EmdPt<V>{(V)0, (V)0, (V)0, (V)0};
    }
  };
  // UB points of the chunk, the u-th at slot ix(u), in increasing slots.
  // ZT: with the zero tests (the exponentials of a batch whose terms all
  // vanish are skipped; float16's never vanish); returns whether a test
  // skipped anything.
  auto batch = [&](auto ix, auto ucnt, auto ztc) -> bool {
    constexpr int UB = decltype(ucnt)::value;
    constexpr bool ZT = decltype(ztc)::value && !std::is_same<T, half_t>::value;
    EmdPt<V> pt[UB];
    V pb[UB];
    V d[UB];
    bool nza = !ZT, nzb = !ZT;
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      pt[u] = s_pt[w][ix(u)];
      if constexpr (NS == 2) pb[u] = s_wb[w][ix(u)];
      d[u] = sq3(pt[u].x - x, pt[u].y - y, pt[u].z - z);
      if constexpr (ZT) {
        nza |= !(d[u] > ta);  // NaN counts as non-zero
        if constexpr (NS == 2) nzb |= !(d[u] > tb);
      }
    }
    bool skipped = false;
    if constexpr (NS == 2 && std::is_same<T, float>::value) {
      if (pow4) {
        // la = 4 lb < 0, so la d <= lb d: a batch whose lb terms all vanish
        // has vanishing la terms too, and both exponentials share one
        // reduction (the same values as two emd_e calls)
        if (!ZT || __builtin_amdgcn_ballot_w64(nzb) != 0) {
          if (!ZT || __builtin_amdgcn_ballot_w64(nza) != 0) {
#pragma unroll
            for (int u = 0; u < UB; ++u) {
              V e1, e4;
              emd_exp_x4(lb * d[u], e1, e4);
              sb = emd_fma(e1, pb[u], sb);
              sa = emd_fma(e4, pt[u].w, sa);
            }
          } else {
#pragma unroll
            for (int u = 0; u < UB; ++u) sb = emd_fma(emd_e<T>(lb, d[u]), pb[u], sb);
            skipped = true;
          }
        } else {
          skipped = true;
        }
        return skipped;
      }
    }
    if (!ZT || __builtin_amdgcn_ballot_w64(nza) != 0) {
#pragma unroll
      for (int u = 0; u < UB; ++u) sa = emd_fma(emd_e<T>(la, d[u]), pt[u].w, sa);
    } else {
      skipped = true;
    }
    if constexpr (NS == 2) {
      if (!ZT || __builtin_amdgcn_ballot_w64(nzb) != 0) {
#pragma unroll
        for (int u = 0; u < UB; ++u) sb = emd_fma(emd_e<T>(lb, d[u]), pb[u], sb);
      } else {
        skipped = true;
      }
    }
    return skipped;
  };
  // Unpruned sweeps keep the zero tests while they pay: after a chunk in
  // which no batch vanished, the rest of the wave's share is summed without
  // them (the same terms; a vanishing term is +0 either way).
  bool zt = true;
  if (q0 < q1) fetch(q0);
  for (int c0 = q0; c0 < q1; c0 += C) {
    // the previous chunk's reads were issued before this write (LDS runs a
    // wave's operations in order), so one slice per wave suffices
    s_pt[w][lane] = nr;
    if constexpr (NS == 2) s_wb[w][lane] = nb;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int cn = min(C, q1 - c0);
    if constexpr (!PR) {
      if (c0 + C < q1) fetch(c0 + C);
      int u0 = 0;
      if (zt) {
        bool skipped = false;
        for (; u0 + U <= cn; u0 += U)
          skipped |= batch([u0](int u) { return u0 + u; }, std::integral_constant<int, U>{},
                           std::true_type{});
        for (; u0 < cn; ++u0)
          skipped |= batch([u0](int) { return u0; }, std::integral_constant<int, 1>{},
                           std::true_type{});
        zt = skipped;
      } else {
        for (; u0 + U <= cn; u0 += U)
          batch([u0](int u) { return u0 + u; }, std::integral_constant<int, U>{},
                std::false_type{});
        for (; u0 < cn; ++u0)
          batch([u0](int) { return u0; }, std::integral_constant<int, 1>{}, std::false_type{});
      }
      __builtin_amdgcn_wave_barrier();
      continue;
    }
    const uint64_t all = cn == C ? ~0ull : (1ull << cn) - 1;
    uint64_t near = all;
    if (prune) {  // lane i tests point c0 + i of the chunk, still in nr
      V g[3];
      const V pc[3] = {nr.x, nr.y, nr.z};
#pragma unroll
      for (int c = 0; c < 3; ++c) {
        const V a = olo[c] - pc[c], e = pc[c] - ohi[c];
        g[c] = a > e ? a : e;
        g[c] = g[c] > (V)0 ? g[c] : (V)0;
      }
      const V lb2 = g[0] * g[0] + g[1] * g[1] + g[2] * g[2];
      const bool pf = __builtin_isfinite(pc[0]) && __builtin_isfinite(pc[1]) &&
                      __builtin_isfinite(pc[2]);
      near &= __builtin_amdgcn_ballot_w64(!(lb2 > reach) || !pf);
    }
    if (c0 + C < q1) fetch(c0 + C);
    const int nn = __builtin_popcountll(near);
    if (nn + U > cn) {  // (nearly) every point: consecutive slots
      int u0 = 0;
      for (; u0 + U <= cn; u0 += U)
        batch([u0](int u) { return u0 + u; }, std::integral_constant<int, U>{}, std::true_type{});
      for (; u0 < cn; ++u0)
        batch([u0](int) { return u0; }, std::integral_constant<int, 1>{}, std::true_type{});
    } else {  // the near points only, in increasing slots
      auto take = [&](auto ucnt) {
        constexpr int UB = decltype(ucnt)::value;
        int sl[UB];
#pragma unroll
        for (int u = 0; u < UB; ++u) {
          sl[u] = __builtin_ctzll(near);
          near &= near - 1;
        }
        batch([&sl](int u) { return sl[u]; }, ucnt, std::true_type{});
      };
      int r = nn;
      for (; r >= U; r -= U) take(std::integral_constant<int, U>{});
      if (r >= 4) {
        take(std::integral_constant<int, 4>{});
        r -= 4;
      }
      if (r >= 2) {
        take(std::integral_constant<int, 2>{});
        r -= 2;
      }
      if (r >= 1) take(std::integral_constant<int, 1>{});
    }
    __builtin_amdgcn_wave_barrier();
  }
  if (w > 0) {
    s_part[0][w - 1][lane] = sa;
    if constexpr (NS == 2) s_part[NS - 1][w - 1][lane] = sb;
  }
  __syncthreads();
  if (w == 0) {  // wave 0's sum, then waves 1 .. NW-1 in order
#pragma unroll
    for (int v = 0; v < NW - 1; ++v) {
      sa += s_part[0][v][lane];
      if constexpr (NS == 2) sb += s_part[NS - 1][v][lane];
    }
    sums[0] = sa;
    if constexpr (NS == 2) sums[1] = sb;
  }
}

// Step s = 0..10 over the xyz1 points: pass 3 of level s-1 (s >= 1), then
// pass 1 of level s (s <= 9).  MODE 1: pass 1 only; 2: pass 3 only; 3: both.
template <typename T, int MODE, bool PR>
__global__ __launch_bounds__(EMD_SWEEP_THREADS) void emd_rows_kernel(
    const typename EmdV<T>::type* __restrict__ p1, const typename EmdV<T>::type* __restrict__ p2,
    const typename EmdV<T>::type* __restrict__ remr, const typename EmdV<T>::type* __restrict__ rr,
    typename EmdV<T>::type* __restrict__ reml, typename EmdV<T>::type* __restrict__ rl,
    const int* __restrict__ ord1, int n, int m, int s) {
  typedef typename EmdV<T>::type V;
  const int64_t b = blockIdx.y;
  const int lane = lane_id();
  const int pos = blockIdx.x * 64 + lane;
  const int k = pos < n ? ord1[b * n + pos] : n;  // this lane's xyz1 point
  V x = (V)0, y = (V)0, z = (V)0;
  if (k < n) {
    x = p1[(b * n + k) * 4];
    y = p1[(b * n + k) * 4 + 1];
    z = p1[(b * n + k) * 4 + 2];
  }
  const V* other = p2 + b * m * 4;
  const V* w3 = rr + (b * EMD_LEVELS + (s >= 1 ? s - 1 : 0)) * m;  // ratioR of level s-1
  const V* w1 = remr + b * m;
  V sums[2];
  const bool own = k < n;
  if constexpr (MODE == 1)
    emd_sweep<T, 1, PR>(other, m, own, x, y, z, emd_level<V>(s), w1, (V)0, w1, sums);
  if constexpr (MODE == 2)
    emd_sweep<T, 1, PR>(other, m, own, x, y, z, emd_level<V>(s - 1), w3, (V)0, w3, sums);
  if constexpr (MODE == 3)
    emd_sweep<T, 2, PR>(other, m, own, x, y, z, emd_level<V>(s - 1), w3, emd_level<V>(s), w1,
                        sums);
  if (wave_id() != 0 || k >= n) return;
  const V eps = emd_eps<T, V>();
  V rem = reml[b * n + k];
  if constexpr (MODE != 1) {  // emd.cu:177-178 (sum_l w = ratioL * sum_l e * ratioR)
    const V ratl = rl[(b * EMD_LEVELS + (s - 1)) * n + k];
    rem = emd_st<T, V>(emd_max0(rem - ratl * sums[0]));
    reml[b * n + k] = rem;
  }
  if constexpr (MODE != 2) {  // emd.cu:88-95
    const V suml = eps + sums[MODE == 3 ? 1 : 0];
    rl[(b * EMD_LEVELS + s) * n + k] = emd_st<T, V>(rem / (suml + eps));
  }
}

// Pass 2 of level t over the xyz2 points (emd.cu:98-138).
template <typename T, bool PR>
__global__ __launch_bounds__(EMD_SWEEP_THREADS) void emd_cols_kernel(
    const typename EmdV<T>::type* __restrict__ p1, const typename EmdV<T>::type* __restrict__ p2,
    const typename EmdV<T>::type* __restrict__ rl, typename EmdV<T>::type* __restrict__ remr,
    typename EmdV<T>::type* __restrict__ rr, const int* __restrict__ ord2, int n, int m, int t) {
  typedef typename EmdV<T>::type V;
  const int64_t b = blockIdx.y;
  const int lane = lane_id();
  const int pos = blockIdx.x * 64 + lane;
  const int l = pos < m ? ord2[b * m + pos] : m;  // this lane's xyz2 point
  V x = (V)0, y = (V)0, z = (V)0;
  if (l < m) {
    x = p2[(b * m + l) * 4];
    y = p2[(b * m + l) * 4 + 1];
    z = p2[(b * m + l) * 4 + 2];
  }
  // d(k,l) takes the differences p2 - p1 as the rows pass does; squaring
  // makes the sign irrelevant, so the same values result.
  V sums[2];
  emd_sweep<T, 1, PR>(p1 + b * n * 4, n, l < m, x, y, z, emd_level<V>(t),
                      rl + (b * EMD_LEVELS + t) * n, (V)0, nullptr, sums);
  if (wave_id() != 0 || l >= m) return;
  const V eps = emd_eps<T, V>();
  const V rem = remr[b * m + l];
  const V sumr = sums[0] * rem;
  const V cons = emd_min1(rem / (sumr + eps));
  rr[(b * EMD_LEVELS + t) * m + l] = emd_st<T, V>(cons * rem);
  remr[b * m + l] = emd_st<T, V>(emd_max0(rem - sumr));
}

// match[l][k] over the ten levels, written once, and matchcost's partial sum.
template <typename T>
__global__ __launch_bounds__(EMD_THREADS) void emd_match_kernel(
    const typename EmdV<T>::type* __restrict__ p1, const typename EmdV<T>::type* __restrict__ p2,
    const typename EmdV<T>::type* __restrict__ rl, const typename EmdV<T>::type* __restrict__ rr,
    int n, int m, T* __restrict__ match, typename EmdV<T>::type* __restrict__ cpart) {
  typedef typename EmdV<T>::type V;
  __shared__ V s_red[EMD_THREADS / 64];
  const int64_t b = blockIdx.z;
  const int k = blockIdx.x * EMD_THREADS + threadIdx.x;
  const bool own = k < n;
  const int kk = own ? k : n - 1;
  const V x = p1[(b * n + kk) * 4], y = p1[(b * n + kk) * 4 + 1], z = p1[(b * n + kk) * 4 + 2];
  V r[EMD_LEVELS];
#pragma unroll
  for (int t = 0; t < EMD_LEVELS; ++t) r[t] = rl[(b * EMD_LEVELS + t) * n + kk];
  const int l0 = blockIdx.y * EMD_MATCH_ROWS;
  const int l1 = min(m, l0 + EMD_MATCH_ROWS);
  const V* q = p2 + b * m * 4;
  const V* rrb = rr + b * EMD_LEVELS * m;
  V cs = (V)0;
  for (int l = l0; l < l1; ++l) {
    const V d = sq3(q[4 * l] - x, q[4 * l + 1] - y, q[4 * l + 2] - z);
    V mt = (V)0;
    auto add = [&](int t, V e) {
      const V w = (e * r[t]) * rrb[t * m + l];  // emd.cu:170
      mt = emd_st<T, V>(mt + emd_st<T, V>(w));  // emd.cu:171
    };
    if constexpr (std::is_same<T, float>::value) {
      // levels 2i and 2i+1 (a factor 4 apart) share one argument reduction;
      // the additions stay in level order.  When only the steeper level
      // vanishes in every lane its terms are exactly +0 and leave mt as is.
#pragma unroll
      for (int t = 0; t < EMD_LEVELS - 2; t += 2) {
        if (emd_wave_zero<T>(emd_level<V>(t + 1), d)) continue;  // both levels vanish
        V e1, e4;
        emd_exp_x4(emd_level<V>(t + 1) * d, e1, e4);
        add(t, e4);
        add(t + 1, e1);
      }
#pragma unroll
      for (int t = EMD_LEVELS - 2; t < EMD_LEVELS; ++t)
        if (!emd_wave_zero<T>(emd_level<V>(t), d)) add(t, emd_e<T>(emd_level<V>(t), d));
    } else {
#pragma unroll
      for (int t = 0; t < EMD_LEVELS; ++t) {
        if (emd_wave_zero<T>(emd_level<V>(t), d)) continue;  // w = +0: mt + 0 == mt
        add(t, emd_e<T>(emd_level<V>(t), d));
      }
    }
    if (own) match[(b * m + l) * (int64_t)n + k] = (T)mt;
    cs = emd_fma(d, mt, cs);  // emd.cu:212-213
  }
  cs = own ? cs : (V)0;
  cs = wave_sum(cs);
  if (lane_id() == 0) s_red[wave_id()] = cs;
  __syncthreads();
  if (threadIdx.x == 0)
    cpart[(b * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x] =
        ((s_red[0] + s_red[1]) + s_red[2]) + s_red[3];
}

// cost[b] = the sum of the cloud's partials, in a fixed order.
template <typename T>
__global__ __launch_bounds__(EMD_THREADS) void emd_cost_kernel(
    const typename EmdV<T>::type* __restrict__ cpart, int parts, T* __restrict__ cost) {
  typedef typename EmdV<T>::type V;
  __shared__ V s_red[EMD_THREADS / 64];
  const int64_t b = blockIdx.x;
  V s = (V)0;
  for (int i = threadIdx.x; i < parts; i += EMD_THREADS) s += cpart[b * parts + i];
  s = wave_sum(s);
  if (lane_id() == 0) s_red[wave_id()] = s;
  __syncthreads();
  if (threadIdx.x == 0)
    cost[b] = (T)emd_st<T, V>(((s_red[0] + s_red[1]) + s_red[2]) + s_red[3]);
}

template <typename T>
__global__ void emd_zero_kernel(T* __restrict__ p, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) p[i] = (T)0;
}

// ---------------------------------------------------------------- backward

// Both gradients' partials in one pass over match (emd.cu:234-303):
//   grad_xyz1[k] = grad_cost * sum_l (p1_k - p2_l) * 2 match[l][k]
//   grad_xyz2[l] = grad_cost * sum_k (p2_l - p1_k) * 2 match[l][k]
// Workgroup (column tile of 4 * 64 columns, row tile of EMD_G1_ROWS rows,
// cloud): lane j of every wave holds columns 4j .. 4j + 3 of the tile (one
// 4-wide load a row), and wave w takes rows w, w + 4, ... of the row tile.
// A column's sum over the wave's rows stays in registers, the waves' sums
// added in wave order at the end (grad_xyz1 partials per row tile); a row's
// sum over the tile's columns is reduced across the wave (grad_xyz2 partials
// per column tile).  Every sum has a fixed order.
constexpr int EMD_GT_COLS = 256;
template <typename T>
__global__ __launch_bounds__(EMD_THREADS) void emd_grad_part_kernel(
    const T* __restrict__ xyz1, const T* __restrict__ xyz2, const T* __restrict__ match, int n,
    int m, bool vec, typename EmdV<T>::type* __restrict__ part1,
    typename EmdV<T>::type* __restrict__ part2) {
  typedef typename EmdV<T>::type V;
  typedef T T4 __attribute__((ext_vector_type(4)));
  constexpr int NW = EMD_THREADS / 64;
  __shared__ V s_col[NW - 1][EMD_GT_COLS][3];
  const int64_t b = blockIdx.z;
  const int w = wave_id(), lane = lane_id();
  const int k0 = blockIdx.x * EMD_GT_COLS + 4 * lane;
  const int l0 = blockIdx.y * EMD_G1_ROWS, l1 = min(m, l0 + EMD_G1_ROWS);
  V x1[4], y1[4], z1[4];
  bool okc[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    okc[q] = k0 + q < n;
    const int64_t kk = b * n + (okc[q] ? k0 + q : n - 1);
    x1[q] = (V)xyz1[kk * 3];
    y1[q] = (V)xyz1[kk * 3 + 1];
    z1[q] = (V)xyz1[kk * 3 + 2];
  }
  V ax[4] = {}, ay[4] = {}, az[4] = {};
  for (int l = l0 + w; l < l1; l += NW) {
    const T* __restrict__ row = match + (b * m + l) * (int64_t)n;
    V d[4];
    if (vec) {  // n % 4 == 0 and match aligned: the 4 columns are all in or all out
      const T4 v = okc[0] ? *reinterpret_cast<const T4*>(row + k0) : T4{};
#pragma unroll
      for (int q = 0; q < 4; ++q) d[q] = (V)v[q] * (V)2;
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) d[q] = okc[q] ? (V)row[k0 + q] * (V)2 : (V)0;
    }
    const V x2 = (V)xyz2[(b * m + l) * 3], y2 = (V)xyz2[(b * m + l) * 3 + 1],
            z2 = (V)xyz2[(b * m + l) * 3 + 2];
    V rx = (V)0, ry = (V)0, rz = (V)0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (!okc[q]) continue;
      const V dx = x1[q] - x2, dy = y1[q] - y2, dz = z1[q] - z2;
      ax[q] = emd_fma(dx, d[q], ax[q]);
      ay[q] = emd_fma(dy, d[q], ay[q]);
      az[q] = emd_fma(dz, d[q], az[q]);
      rx = emd_fma(-dx, d[q], rx);
      ry = emd_fma(-dy, d[q], ry);
      rz = emd_fma(-dz, d[q], rz);
    }
    rx = wave_total63(rx);
    ry = wave_total63(ry);
    rz = wave_total63(rz);
    if (lane == 63) {
      V* __restrict__ o = part2 + ((b * gridDim.x + blockIdx.x) * m + l) * 3;
      o[0] = rx;
      o[1] = ry;
      o[2] = rz;
    }
  }
  if (w > 0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      s_col[w - 1][4 * lane + q][0] = ax[q];
      s_col[w - 1][4 * lane + q][1] = ay[q];
      s_col[w - 1][4 * lane + q][2] = az[q];
    }
  }
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (!okc[q]) continue;
#pragma unroll
      for (int v = 0; v < NW - 1; ++v) {
        ax[q] += s_col[v][4 * lane + q][0];
        ay[q] += s_col[v][4 * lane + q][1];
        az[q] += s_col[v][4 * lane + q][2];
      }
      V* __restrict__ o = part1 + ((b * gridDim.y + blockIdx.y) * n + k0 + q) * 3;
      o[0] = ax[q];
      o[1] = ay[q];
      o[2] = az[q];
    }
  }
}

// grad_xyz1 (blockIdx.z = 0: n points, nchunk row-tile partials) and
// grad_xyz2 (blockIdx.z = 1: m points, ncol column-tile partials):
// grad_cost[b] times the sum of the partials, added in order
template <typename T>
__global__ __launch_bounds__(EMD_THREADS) void emd_grad_final_kernel(
    const T* __restrict__ grad_cost, const typename EmdV<T>::type* __restrict__ part1,
    const typename EmdV<T>::type* __restrict__ part2, int n, int m, int nchunk, int ncol,
    T* __restrict__ grad1, T* __restrict__ grad2) {
  typedef typename EmdV<T>::type V;
  const int64_t b = blockIdx.y;
  const bool second = blockIdx.z != 0;
  const int cnt = second ? m : n, parts = second ? ncol : nchunk;
  const V* __restrict__ part = second ? part2 : part1;
  T* __restrict__ grad = second ? grad2 : grad1;
  const int k = blockIdx.x * EMD_THREADS + threadIdx.x;
  if (k >= cnt) return;
  V a[3] = {(V)0, (V)0, (V)0};
  for (int c = 0; c < parts; ++c) {
    const V* o = part + ((b * parts + c) * cnt + k) * 3;
    a[0] += o[0];
    a[1] += o[1];
    a[2] += o[2];
  }
  const V g = (V)grad_cost[b];
#pragma unroll
  for (int c = 0; c < 3; ++c) grad[(b * cnt + k) * 3 + c] = (T)(a[c] * g);
}

// ---------------------------------------------------------------- host side

template <typename T>
int emd_fwd_impl(const void* xyz1, const void* xyz2, int64_t B, int64_t n, int64_t m, void* cost,
                 void* match, char* ws, hipStream_t s) {
  typedef typename EmdV<T>::type V;
  const EmdLayout L = emd_layout<V>(B, n, m);
  V* p1 = (V*)(ws + L.p1);
  V* p2 = (V*)(ws + L.p2);
  V* reml = (V*)(ws + L.reml);
  V* remr = (V*)(ws + L.remr);
  V* rl = (V*)(ws + L.rl);
  V* rr = (V*)(ws + L.rr);
  V* cp = (V*)(ws + L.cost);
  int* ord1 = (int*)(ws + L.ord1);
  int* ord2 = (int*)(ws + L.ord2);
  // emd.cu:21-28: float(n)/m
  const float mult_l = n >= m ? 1.0f : (float)m / (float)n;
  const float mult_r = n >= m ? (float)n / (float)m : 1.0f;
  const int nn = (int)n, mm = (int)m;
  const unsigned bb = (unsigned)B;
  hipLaunchKernelGGL(emd_prep_kernel<T>, dim3((unsigned)((std::max(n, m) + 255) / 256), bb),
                     dim3(EMD_THREADS), 0, s, (const T*)xyz1, (const T*)xyz2, nn, mm, mult_l, mult_r,
                     p1, p2, reml, remr);
  {  // the k-d order for clouds that fit it, else the Morton order
    const bool kd1 = n <= EMD_KD_MAX, kd2 = m <= EMD_KD_MAX;
    auto order = [&](bool kd, unsigned clouds, int first) {
      if (kd)
        hipLaunchKernelGGL(emd_kd_order_kernel<T>, dim3(bb, clouds), dim3(EMD_ORDER_THREADS), 0, s,
                           (const T*)xyz1, (const T*)xyz2, nn, mm, ord1, ord2, first);
      else
        hipLaunchKernelGGL(emd_order_kernel<T>, dim3(bb, clouds), dim3(EMD_ORDER_THREADS), 0, s,
                           (const T*)xyz1, (const T*)xyz2, nn, mm, ord1, ord2, first);
    };
    if (kd1 == kd2) {
      order(kd1, 2, 0);
    } else {
      order(kd1, 1, 0);
      order(kd2, 1, 1);
    }
  }
  const dim3 grow((unsigned)((n + 63) / 64), bb), gcol((unsigned)((m + 63) / 64), bb);
  // Far points are left out of the steep levels' sweeps (levels -4^7 ..
  // -4^3, those whose zero distance reaches a small part of a cloud of unit
  // scale); float16's exponentials never vanish.
  constexpr bool prunable = !std::is_same<T, half_t>::value;
  constexpr int EMD_PRUNE_STEPS = 5;
#define EMD_ROWS(MODE, PR)                                                                 \
  hipLaunchKernelGGL((emd_rows_kernel<T, MODE, PR>), grow, dim3(EMD_SWEEP_THREADS), 0, s, p1, \
                     p2, remr, rr, reml, rl, ord1, nn, mm, st)
#define EMD_COLS(PR)                                                                     \
  hipLaunchKernelGGL((emd_cols_kernel<T, PR>), gcol, dim3(EMD_SWEEP_THREADS), 0, s, p1, p2, rl, \
                     remr, rr, ord2, nn, mm, st)
  for (int st = 0; st <= EMD_LEVELS; ++st) {
    const bool pr = prunable && st < EMD_PRUNE_STEPS;
    if (st == 0) {
      if (pr) EMD_ROWS(1, prunable);
      else EMD_ROWS(1, false);
    } else if (st == EMD_LEVELS) {
      EMD_ROWS(2, false);
    } else {
      if (pr) EMD_ROWS(3, prunable);
      else EMD_ROWS(3, false);
    }
    if (st < EMD_LEVELS) {
      if (pr) EMD_COLS(prunable);
      else EMD_COLS(false);
    }
  }
#undef EMD_ROWS
#undef EMD_COLS
  hipLaunchKernelGGL(emd_match_kernel<T>, dim3((unsigned)L.gx, (unsigned)L.gy, bb),
                     dim3(EMD_THREADS), 0, s, p1, p2, rl, rr, nn, mm, (T*)match, cp);
  hipLaunchKernelGGL(emd_cost_kernel<T>, dim3(bb), dim3(EMD_THREADS), 0, s, cp, L.gx * L.gy,
                     (T*)cost);
  return check_launch("tpo_emd_fwd");
}

template <typename T>
int emd_bwd_impl(const void* grad_cost, const void* xyz1, const void* xyz2, const void* match,
                 int64_t B, int64_t n, int64_t m, void* grad1, void* grad2, char* ws,
                 hipStream_t s) {
  typedef typename EmdV<T>::type V;
  const EmdLayout L = emd_layout<V>(B, n, m);
  V* part1 = (V*)(ws + L.g1);
  V* part2 = (V*)(ws + L.g2);
  const int nn = (int)n, mm = (int)m;
  const unsigned bb = (unsigned)B;
  const bool vec = (n % 4) == 0 && (reinterpret_cast<uintptr_t>(match) % (4 * sizeof(T))) == 0;
  hipLaunchKernelGGL(emd_grad_part_kernel<T>, dim3((unsigned)L.gx, (unsigned)L.nchunk, bb),
                     dim3(EMD_THREADS), 0, s, (const T*)xyz1, (const T*)xyz2, (const T*)match, nn,
                     mm, vec, part1, part2);
  hipLaunchKernelGGL(emd_grad_final_kernel<T>,
                     dim3((unsigned)((std::max(n, m) + EMD_THREADS - 1) / EMD_THREADS), bb, 2),
                     dim3(EMD_THREADS), 0, s, (const T*)grad_cost, part1, part2, nn, mm, L.nchunk,
                     L.gx, (T*)grad1, (T*)grad2);
  return check_launch("tpo_emd_bwd");
}

template <typename T>
void emd_zero(void* p, int64_t count, hipStream_t s) {
  if (count <= 0) return;
  hipLaunchKernelGGL(emd_zero_kernel<T>, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s,
                     (T*)p, count);
}

// Clouds per launch: the kernels put the cloud index in grid y or z.
constexpr int64_t EMD_CLOUDS_PER_LAUNCH = 65535;

// Launch sequences for any B: clouds in chunks, reusing the workspace (sized
// for B, so large enough for every chunk) in stream order.
template <typename T>
int emd_fwd_chunks(const void* xyz1, const void* xyz2, int64_t B, int64_t n, int64_t m, void* cost,
                   void* match, char* ws, hipStream_t s) {
  for (int64_t b0 = 0; b0 < B; b0 += EMD_CLOUDS_PER_LAUNCH) {
    const int64_t bc = std::min(EMD_CLOUDS_PER_LAUNCH, B - b0);
    if (int rc = emd_fwd_impl<T>((const T*)xyz1 + b0 * n * 3, (const T*)xyz2 + b0 * m * 3, bc, n,
                                 m, (T*)cost + b0, (T*)match + b0 * m * n, ws, s))
      return rc;
  }
  return TPO_OK;
}
template <typename T>
int emd_bwd_chunks(const void* grad_cost, const void* xyz1, const void* xyz2, const void* match,
                   int64_t B, int64_t n, int64_t m, void* grad1, void* grad2, char* ws,
                   hipStream_t s) {
  for (int64_t b0 = 0; b0 < B; b0 += EMD_CLOUDS_PER_LAUNCH) {
    const int64_t bc = std::min(EMD_CLOUDS_PER_LAUNCH, B - b0);
    if (int rc = emd_bwd_impl<T>((const T*)grad_cost + b0, (const T*)xyz1 + b0 * n * 3,
                                 (const T*)xyz2 + b0 * m * 3, (const T*)match + b0 * m * n, bc, n,
                                 m, (T*)grad1 + b0 * n * 3, (T*)grad2 + b0 * m * 3, ws, s))
      return rc;
  }
  return TPO_OK;
}

int emd_check_sizes(const char* what, int64_t B, int64_t n, int64_t m) {
  if (B < 0 || n < 0 || m < 0 || B >= ((int64_t)1 << 31) || n >= ((int64_t)1 << 30) ||
      m >= ((int64_t)1 << 30) || n * m >= ((int64_t)1 << 40))
    return set_error(TPO_ERR_ARG, "%s: bad sizes B=%lld n=%lld m=%lld", what, (long long)B,
                     (long long)n, (long long)m);
  return TPO_OK;
}

}  // namespace
}  // namespace tpo

using namespace tpo;

extern "C" int64_t tpo_emd_workspace_size(int dtype, int64_t B, int64_t n, int64_t m) {
  if (B < 0 || n < 0 || m < 0) return -1;
  if (B == 0 || n == 0 || m == 0) return 0;
  switch (dtype) {
    case TPO_F32:
    case TPO_F16: return emd_layout<float>(B, n, m).total;
    case TPO_F64: return emd_layout<double>(B, n, m).total;
    default: set_error(TPO_ERR_DTYPE, "tpo_emd_workspace_size: unsupported dtype %d", dtype); return -1;
  }
}

extern "C" int tpo_emd_fwd(int dtype, const void* xyz1, const void* xyz2, int64_t B, int64_t n,
                           int64_t m, void* cost, void* match, void* workspace,
                           int64_t workspace_bytes, void* stream) {
  if (int rc = emd_check_sizes("tpo_emd_fwd", B, n, m)) return rc;
  if (dtype != TPO_F32 && dtype != TPO_F64 && dtype != TPO_F16)
    return set_error(TPO_ERR_DTYPE, "tpo_emd_fwd: unsupported dtype %d", dtype);
  hipStream_t s = (hipStream_t)stream;
  if (B == 0) return TPO_OK;
  if (n == 0 || m == 0) {  // emd.cu:313-318: zero cost, empty match
    if (dtype == TPO_F64) emd_zero<double>(cost, B, s);
    else if (dtype == TPO_F32) emd_zero<float>(cost, B, s);
    else emd_zero<half_t>(cost, B, s);
    return check_launch("tpo_emd_fwd");
  }
  const int64_t need = tpo_emd_workspace_size(dtype, B, n, m);
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255))
    return set_error(TPO_ERR_WORKSPACE, "tpo_emd_fwd: workspace needs %lld bytes (256-aligned)",
                     (long long)need);
  switch (dtype) {
    case TPO_F32: return emd_fwd_chunks<float>(xyz1, xyz2, B, n, m, cost, match, (char*)workspace, s);
    case TPO_F64: return emd_fwd_chunks<double>(xyz1, xyz2, B, n, m, cost, match, (char*)workspace, s);
    default: return emd_fwd_chunks<half_t>(xyz1, xyz2, B, n, m, cost, match, (char*)workspace, s);
  }
}

extern "C" int tpo_emd_bwd(int dtype, const void* grad_cost, const void* xyz1, const void* xyz2,
                           const void* match, int64_t B, int64_t n, int64_t m, void* grad_xyz1,
                           void* grad_xyz2, void* workspace, int64_t workspace_bytes,
                           void* stream) {
  if (int rc = emd_check_sizes("tpo_emd_bwd", B, n, m)) return rc;
  if (dtype != TPO_F32 && dtype != TPO_F64 && dtype != TPO_F16)
    return set_error(TPO_ERR_DTYPE, "tpo_emd_bwd: unsupported dtype %d", dtype);
  hipStream_t s = (hipStream_t)stream;
  if (B == 0) return TPO_OK;
  if (n == 0 || m == 0) {  // emd.cu:365-369
    if (dtype == TPO_F64) {
      emd_zero<double>(grad_xyz1, B * n * 3, s);
      emd_zero<double>(grad_xyz2, B * m * 3, s);
    } else if (dtype == TPO_F32) {
      emd_zero<float>(grad_xyz1, B * n * 3, s);
      emd_zero<float>(grad_xyz2, B * m * 3, s);
    } else {
      emd_zero<half_t>(grad_xyz1, B * n * 3, s);
      emd_zero<half_t>(grad_xyz2, B * m * 3, s);
    }
    return check_launch("tpo_emd_bwd");
  }
  const int64_t need = tpo_emd_workspace_size(dtype, B, n, m);
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255))
    return set_error(TPO_ERR_WORKSPACE, "tpo_emd_bwd: workspace needs %lld bytes (256-aligned)",
                     (long long)need);
  switch (dtype) {
    case TPO_F32:
      return emd_bwd_chunks<float>(grad_cost, xyz1, xyz2, match, B, n, m, grad_xyz1, grad_xyz2,
                                   (char*)workspace, s);
    case TPO_F64:
      return emd_bwd_chunks<double>(grad_cost, xyz1, xyz2, match, B, n, m, grad_xyz1, grad_xyz2,
                                    (char*)workspace, s);
    default:
      return emd_bwd_chunks<half_t>(grad_cost, xyz1, xyz2, match, B, n, m, grad_xyz1, grad_xyz2,
                                    (char*)workspace, s);
  }
}
