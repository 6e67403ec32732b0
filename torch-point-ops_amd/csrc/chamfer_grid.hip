// chamfer_grid.hip -- Chamfer forward for float and half clouds by exact grid
// search (replaces chamfer_dist_kernel, chamfer.cu:36-167, when the caller
// provides a workspace and both clouds have at least CH_PRUNE_MIN points).
// Half coordinates are held as float copies (exact) for the grid; distances
// are computed in half as the reference does, and the pruning margins cover
// half rounding (CgMargin).
//
// 1. chamfer_grid_sort_kernel, one workgroup per (batch, cloud): the cloud's
//    bounding box, a counting sort of its points into a 32^3 grid of cells
//    (cells in Morton order, so neighbouring cells are mostly close in
//    memory), the sorted points as (x, y, z, original index) and the start of
//    every cell.
// 2. chamfer_grid_search_kernel: one lane per query, queries taken in the
//    sorted (Morton) order of their own cloud so a wave's lanes search nearby
//    cells.  A lane walks Chebyshev rings of cells around its query's cell
//    until it has a candidate (ring 1 nearest cells first, its edge and
//    corner groups skipped whole when a lower bound of their gaps exceeds
//    the best distance), then visits the box of cells that can hold a
//    point within the best distance found (cell assignment is monotone in
//    each coordinate, and the box is widened by 2^-19 relative plus the
//    rounding of its bounds), evaluating every point of a visited cell with
//    the reference formula (chamfer.cu:64-67, same bits) and keeping the
//    smallest (distance, original index) -- the reference's first-index rule.
//    A cell is skipped when a lower bound of its squared distance, rounded
//    down by 2^-20 relative, exceeds the best distance: the reference's float
//    distance of any of its points is then strictly larger (its relative
//    error is <= 5u), so neither a smaller distance nor a tie with a lower
//    index is missed.  Cell boxes are widened by 2^-20 (|lo| + extent) per
//    side, which covers the rounding of the cell assignment.
// 3. Queries with a coordinate that is non-finite or >= 2^60 in magnitude,
//    and every query of a reference cloud holding such a coordinate, are
//    scanned over the whole reference cloud in original order by chunk_scan
//    (the reference's NaN rule included).
// The best (distance, index) pair is one 64-bit key: distances here are
// finite and non-negative, so their bits order like their values.
// Uneven clouds: the search runs at the finest of 32^3, 16^3 and 8^3 cells
// whose mean own-cell occupancy is small; a box stretched by a few far
// points is rebuilt on the remaining points (the cut sides' boundary cells
// unbounded); a cloud still crowded into few cells runs the dense block
// inside the search kernel; a query whose box would hold too many cells
// joins a wave-wide scan of the reference cloud.  Results are identical to
// the reference's in every case; only the work depends on the data.  Each
// wave records the number of points it evaluated
// (tpo_chamfer_pairs_evaluated sums them).
#include <algorithm>

#include "chamfer_common.hpp"
#include "chamfer_dense.hpp"

#pragma clang fp contract(off)

namespace tpo {

constexpr int CG_GRID = 32;  // cells per axis
constexpr int CG_CELLS = CG_GRID * CG_GRID * CG_GRID;
constexpr int CG_CSTRIDE = CG_CELLS + 4;  // cell-start ints per cloud (16-byte rows)
constexpr int CG_WG = 256;    // queries per search workgroup
constexpr int CG_UNROLL = 2;  // points of a cell loaded together
constexpr int CG_OCC = 2;     // mean own-cell occupancy the search resolution aims at

__host__ __device__ inline int64_t cg_pad(int64_t n) { return (n + 63) & ~(int64_t)63; }

// Byte offsets of the workspace regions (all 256-byte aligned).
struct CgLayout {
  int64_t hdr;     // 2B x 16 floats: lo[3], hi[3], cells per unit[3], cell size[3] (32^3),
                   // bad, degenerate, level (search cells are 2^level of them per axis),
                   // cut sides (bit a: axis a cut below, 3 + a: above; the boundary
                   // cells on a cut side are unbounded)
  int64_t pts;     // float4 per padded point: sorted (x, y, z, original index bits)
  int64_t cstart;  // CG_CSTRIDE int32 per cloud: first sorted position of a cell, then n
  int64_t rank;    // int32 per point: rank within its cell (sort scratch)
  int64_t stats;   // int32 per search wave: points evaluated
  int64_t total;
};

static int64_t cg_align(int64_t x) { return (x + 255) & ~(int64_t)255; }

static int64_t cg_grid_size(int64_t B, int64_t N, int64_t M) {
  return B * ((N + CG_WG - 1) / CG_WG + (M + CG_WG - 1) / CG_WG);
}

static CgLayout cg_layout(int64_t B, int64_t N, int64_t M) {
  const int64_t P = cg_pad(N) + cg_pad(M);
  CgLayout L;
  int64_t o = 0;
  L.hdr = o;
  o = cg_align(o + 2 * B * 16 * 4);
  L.pts = o;
  o = cg_align(o + B * P * 16);
  L.cstart = o;
  o = cg_align(o + 2 * B * CG_CSTRIDE * 4);
  L.rank = o;
  o = cg_align(o + B * P * 4);
  L.stats = o;
  o = cg_align(o + cg_grid_size(B, N, M) * (CG_WG / 64) * 4);
  L.total = o;
  return L;
}

__device__ __forceinline__ uint32_t cg_spread(uint32_t v) {  // 5 bits -> every third bit
  v = (v | (v << 8)) & 0x100fu;
  v = (v | (v << 4)) & 0x10c3u;
  v = (v | (v << 2)) & 0x1249u;
  return v;
}

__device__ __forceinline__ int cg_axis_cell(float p, float lo, float sc, int g = CG_GRID) {
  const float f = (p - lo) * sc;
  return is_nan(f) ? 0 : (int)fminf(fmaxf(f, 0.f), (float)(g - 1));
}

__device__ __forceinline__ uint32_t cg_code(int cx, int cy, int cz) {
  return cg_spread((uint32_t)cx) | (cg_spread((uint32_t)cy) << 1) | (cg_spread((uint32_t)cz) << 2);
}

// The histogram is stored with one padding word per 32 cells, so the scan's
// per-thread runs of 32 consecutive cells fall in different LDS banks.
__device__ __forceinline__ int cg_hidx(uint32_t code) { return (int)(code + (code >> 5)); }

// The reference's squared distance (chamfer.cu:64-67) in the input type T,
// from the float copies of T coordinates the workspace holds (exact); the
// result is returned as float (exact).
template <typename T>
__device__ __forceinline__ float cg_dist(const float4& p, const float4& q);
template <>
__device__ __forceinline__ float cg_dist<float>(const float4& p, const float4& q) {
  return sq3((float)(p.x - q.x), (float)(p.y - q.y), (float)(p.z - q.z));
}
template <>
__device__ __forceinline__ float cg_dist<half_t>(const float4& p, const float4& q) {
  return (float)sq3((half_t)((half_t)p.x - (half_t)q.x), (half_t)((half_t)p.y - (half_t)q.y),
                    (half_t)((half_t)p.z - (half_t)q.z));
}

// Pruning margins: a cell whose float lower bound g2 of the exact squared
// distance satisfies g2 * lb - abs > best holds no point whose computed
// distance is <= best, and every point with computed distance <= best lies
// within sqrt((best + abs) * inv) of the query.  float: the computed
// distance is within 5u (u = 2^-24) of the exact one, far inside the 2^-20
// factor.  half: six roundings of relative error <= 2^-11 each, plus the
// absolute error of subnormal intermediates (< 2^-22 in all), so lb is
// below (1 - 2^-20)(1 - 2^-11)^6, inv above (1 - 2^-11)^-6 and abs 2^-20.
template <typename T>
struct CgMargin;
template <>
struct CgMargin<float> {
  static constexpr float lb = 1.f - 0x1p-20f, abs = 0.f, inv = 1.f;
};
template <>
struct CgMargin<half_t> {
  static constexpr float lb = 0.997f, abs = 0x1p-20f, inv = 1.003f;
};

// PPT > 0: every thread keeps its (at most PPT) points in registers across the
// passes (n <= 1024 * PPT); PPT == 0: the passes reload from memory.
template <typename TI, int PPT>
__global__ __launch_bounds__(1024) void chamfer_grid_sort_kernel(
    const TI* __restrict__ xyz1, const TI* __restrict__ xyz2, int N, int M,
    char* __restrict__ ws, CgLayout L, uint32_t* __restrict__ zero) {
  // cell counts, then (PPT > 0) the sorted points staged for a coalesced write
  __shared__ __align__(16) uint32_t cnt[CG_CELLS + CG_CELLS / 32];
  static_assert(sizeof(cnt) >= 1024 * 8 * sizeof(float4), "staging area");
  __shared__ float red[6][16];
  __shared__ uint32_t part[16];
  __shared__ uint32_t s_bad, s_maxc;
  __shared__ float s_sq[3][16];  // per wave: sum of count^2 over the cells of 32^3, 16^3, 8^3
  const int c = blockIdx.x & 1, b = blockIdx.x >> 1;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int n = c ? M : N;
  if (zero && blockIdx.x == 0 && tid == 0) *zero = 0u;
  const int64_t PN = cg_pad(N), PM = cg_pad(M);
  const int64_t base = (int64_t)b * (PN + PM) + (c ? PN : 0);
  const TI* __restrict__ P = (c ? xyz2 : xyz1) + (size_t)b * n * 3;
  float* __restrict__ hdr = reinterpret_cast<float*>(ws + L.hdr) + (size_t)blockIdx.x * 16;
  float4* __restrict__ pts = reinterpret_cast<float4*>(ws + L.pts) + base;
  int32_t* __restrict__ cstart =
      reinterpret_cast<int32_t*>(ws + L.cstart) + (size_t)blockIdx.x * CG_CSTRIDE;
  int32_t* __restrict__ rank = reinterpret_cast<int32_t*>(ws + L.rank) + base;

  constexpr int R = PPT > 0 ? PPT : 1;
  float px[R], py[R], pz[R];
  if constexpr (PPT > 0) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int k = min(tid + 1024 * i, n - 1);  // duplicates of the last point: harmless below
      px[i] = (float)P[3 * k];
      py[i] = (float)P[3 * k + 1];
      pz[i] = (float)P[3 * k + 2];
    }
  }
  auto point = [&](int i, int k, float& x, float& y, float& z) {
    if constexpr (PPT > 0) {
      x = px[i];
      y = py[i];
      z = pz[i];
    } else {
      x = (float)P[3 * k];
      y = (float)P[3 * k + 1];
      z = (float)P[3 * k + 2];
    }
  };
  const int iters = PPT > 0 ? PPT : (n + 1023) / 1024;

  // bounding box (NaN ignored) and the bad flag (non-finite or >= 2^60)
  if (tid == 0) s_bad = s_maxc = 0;
  float lo[3] = {__builtin_inff(), __builtin_inff(), __builtin_inff()};
  float hi[3] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
  uint32_t big = 0;
  for (int i = 0; i < iters; ++i) {
    const int k = tid + 1024 * i;
    if (k >= n) break;
    float v[3];
    point(i, k, v[0], v[1], v[2]);
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      big = max(big, abs_bits(v[a]));
      lo[a] = fminf(lo[a], v[a]);
      hi[a] = fmaxf(hi[a], v[a]);
    }
  }
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      lo[a] = fminf(lo[a], __shfl_xor(lo[a], m));
      hi[a] = fmaxf(hi[a], __shfl_xor(hi[a], m));
    }
  if (lane == 0)
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      red[a][w] = lo[a];
      red[3 + a][w] = hi[a];
    }
  for (int k = tid; k < (CG_CELLS + CG_CELLS / 32) / 4; k += 1024)
    reinterpret_cast<uint4*>(cnt)[k] = make_uint4(0u, 0u, 0u, 0u);
  __syncthreads();
  if (big >= CH_BIG) atomicOr(&s_bad, 1u);
  float glo[3], ghi[3], gs[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    float x = __builtin_inff(), z = -__builtin_inff();
    for (int v = 0; v < 16; ++v) {
      x = fminf(x, red[a][v]);
      z = fmaxf(z, red[3 + a][v]);
    }
    if (!is_finite(x) || !is_finite(z)) x = z = 0.f;  // empty or all-NaN axis
    glo[a] = x;
    ghi[a] = z;
    const float ext = z - x;
    gs[a] = (ext > 0.f && is_finite(ext)) ? (float)CG_GRID / ext : 0.f;
  }
  auto code_of = [&](float x, float y, float z) {
    return cg_code(cg_axis_cell(x, glo[0], gs[0]), cg_axis_cell(y, glo[1], gs[1]),
                   cg_axis_cell(z, glo[2], gs[2]));
  };
  uint32_t rk[R], hx[R];  // PPT > 0: rank within the cell, histogram slot of the cell
  // the cell histogram; every point's rank within its cell, and the largest
  // cell count (the atomics' returned ranks, maximised)
  auto histogram = [&]() {
    uint32_t mr = 0;
    for (int i = 0; i < iters; ++i) {
      const int k = tid + 1024 * i;
      if (k >= n) break;
      float x, y, z;
      point(i, k, x, y, z);
      const int h = cg_hidx(code_of(x, y, z));
      const uint32_t r = atomicAdd(&cnt[h], 1u);
      mr = max(mr, r + 1);
      if constexpr (PPT > 0) {
        rk[i] = r;
        hx[i] = (uint32_t)h;
      } else {
        rank[k] = (int32_t)r;
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) mr = max(mr, (uint32_t)__shfl_xor((int)mr, m));
    if (lane == 0) atomicMax(&s_maxc, mr);
    __syncthreads();
  };
  histogram();
  // A degenerate grid (a cell of more than max(256, n / 32) points) usually
  // comes from a few far points stretching the box.  Per axis, the sparse
  // tails (bins of the 32 that together hold at most n / 1024 points,
  // walked in from each end) are cut off: the box
  // becomes the extent of the remaining points, the cut points fall into the
  // boundary cells (cell assignment clamps), and those boundary cells are
  // unbounded on the cut side for the search's pruning (header word 15).
  const float occ_lim = (float)max(256, n / 32) * (float)n;
  uint32_t trim = 0;  // bit a: axis a cut below; bit 3 + a: cut above
  if (s_maxc > (uint32_t)max(256, n / 32)) {
    for (int k = tid; k < 96; k += 1024) cnt[k] = 0u;
    __syncthreads();
    for (int i = 0; i < iters; ++i) {
      const int k = tid + 1024 * i;
      if (k >= n) break;
      float v[3];
      point(i, k, v[0], v[1], v[2]);
#pragma unroll
      for (int a = 0; a < 3; ++a) atomicAdd(&cnt[32 * a + cg_axis_cell(v[a], glo[a], gs[a])], 1u);
    }
    __syncthreads();
    int blo[3], bhi[3];
    const uint32_t thr = (uint32_t)n >> 10;
#pragma unroll
    for (int a = 0; a < 3; ++a) {  // every thread reads the same 32 counts
      uint32_t cum = 0;
      int lb = 0;
      while (lb < CG_GRID - 1 && cum + cnt[32 * a + lb] <= thr) cum += cnt[32 * a + lb++];
      cum = 0;
      int ub = CG_GRID - 1;
      while (ub > lb && cum + cnt[32 * a + ub] <= thr) cum += cnt[32 * a + ub--];
      blo[a] = gs[a] > 0.f ? lb : 0;
      bhi[a] = gs[a] > 0.f ? ub : CG_GRID - 1;
    }
    // extent of the points inside the kept bins, per axis
    float tl[3] = {__builtin_inff(), __builtin_inff(), __builtin_inff()};
    float th[3] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
    for (int i = 0; i < iters; ++i) {
      const int k = tid + 1024 * i;
      if (k >= n) break;
      float v[3];
      point(i, k, v[0], v[1], v[2]);
#pragma unroll
      for (int a = 0; a < 3; ++a) {
        const int cb = cg_axis_cell(v[a], glo[a], gs[a]);
        if (cb >= blo[a] && cb <= bhi[a]) {
          tl[a] = fminf(tl[a], v[a]);
          th[a] = fmaxf(th[a], v[a]);
        }
      }
    }
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) {
        tl[a] = fminf(tl[a], __shfl_xor(tl[a], m));
        th[a] = fmaxf(th[a], __shfl_xor(th[a], m));
      }
    __syncthreads();
    if (lane == 0)
#pragma unroll
      for (int a = 0; a < 3; ++a) {
        red[a][w] = tl[a];
        red[3 + a][w] = th[a];
      }
    __syncthreads();
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      float x = __builtin_inff(), z = -__builtin_inff();
      for (int v = 0; v < 16; ++v) {
        x = fminf(x, red[a][v]);
        z = fmaxf(z, red[3 + a][v]);
      }
      if (gs[a] > 0.f && is_finite(x) && is_finite(z)) {
        if (x > glo[a]) trim |= 1u << a;
        if (z < ghi[a]) trim |= 8u << a;
        glo[a] = x;
        ghi[a] = z;
        const float ext = z - x;
        gs[a] = (ext > 0.f && is_finite(ext)) ? (float)CG_GRID / ext : 0.f;
      }
    }
    __syncthreads();
    // rebuild the cell histogram (on the new box; its first counters held
    // the bins above either way)
    for (int k = tid; k < (CG_CELLS + CG_CELLS / 32) / 4; k += 1024)
      reinterpret_cast<uint4*>(cnt)[k] = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();
    histogram();
  }
  {  // exclusive scan of the cell counts, CPT consecutive cells per thread
    constexpr int CPT = CG_CELLS / 1024;
    uint32_t v[CPT], sum = 0;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      v[i] = cnt[cg_hidx(tid * CPT + i)];
      sum += v[i];
    }
    {
      // sums of count^2 over the cells of 32^3, 16^3 and 8^3 (Morton order
      // nests them: 8 consecutive cells form a 16^3 cell, this thread's 32
      // and its neighbour's an 8^3 cell), in float, reduced in a fixed order
      float sq0 = 0.f, sq1 = 0.f;
#pragma unroll
      for (int i = 0; i < CPT; i += 8) {
        uint32_t c8 = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          sq0 = __builtin_fmaf((float)v[i + k], (float)v[i + k], sq0);
          c8 += v[i + k];
        }
        sq1 = __builtin_fmaf((float)c8, (float)c8, sq1);
      }
      const float c64 = (float)(sum + (uint32_t)__shfl_xor((int)sum, 1));
      float sq2 = (lane & 1) ? 0.f : c64 * c64;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        sq0 += __shfl_xor(sq0, o);
        sq1 += __shfl_xor(sq1, o);
        sq2 += __shfl_xor(sq2, o);
      }
      if (lane == 0) {
        s_sq[0][w] = sq0;
        s_sq[1][w] = sq1;
        s_sq[2][w] = sq2;
      }
    }
    uint32_t incl = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t o = (uint32_t)__shfl_up((int)incl, d);
      if (lane >= d) incl += o;
    }
    if (lane == 63) part[w] = incl;
    __syncthreads();
    uint32_t run = incl - sum;
    for (int v2 = 0; v2 < w; ++v2) run += part[v2];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      cnt[cg_hidx(tid * CPT + i)] = run;
      run += v[i];
    }
    if (tid == 1023) cstart[CG_CELLS] = (int32_t)run;
  }
  __syncthreads();
  for (int k = tid; k < CG_CELLS / 4; k += 1024) {  // coalesced, 4 cells per store
    const int c0 = cg_hidx(4 * k);  // the 4 cells share one padded run of 32
    reinterpret_cast<int4*>(cstart)[k] =
        make_int4((int)cnt[c0], (int)cnt[c0 + 1], (int)cnt[c0 + 2], (int)cnt[c0 + 3]);
  }
  if constexpr (PPT > 0) {
    // sorted positions into registers; once every read of the counts is done
    // the points are placed in LDS and written out in order, coalesced
    uint32_t at[R];
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int k = tid + 1024 * i;
      at[i] = k < n ? cnt[hx[i]] + rk[i] : 0u;
    }
    __syncthreads();
    float4* __restrict__ stage = reinterpret_cast<float4*>(cnt);
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int k = tid + 1024 * i;
      if (k < n) stage[at[i]] = make_float4(px[i], py[i], pz[i], __int_as_float(k));
    }
    __syncthreads();
    for (int pos = tid; pos < cg_pad(n); pos += 1024)
      pts[pos] = pos < n ? stage[pos] : make_float4(0.f, 0.f, 0.f, __int_as_float(-1));
  } else {
    for (int i = 0; i < iters; ++i) {
      const int k = tid + 1024 * i;
      if (k >= n) break;
      float x, y, z;
      point(i, k, x, y, z);
      pts[cnt[cg_hidx(code_of(x, y, z))] + (uint32_t)rank[k]] =
          make_float4(x, y, z, __int_as_float(k));
    }
    for (int pos = n + tid; pos < cg_pad(n); pos += 1024)
      pts[pos] = make_float4(0.f, 0.f, 0.f, __int_as_float(-1));
  }
  if (tid == 0) {
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      hdr[a] = glo[a];
      hdr[3 + a] = ghi[a];
      hdr[6 + a] = gs[a];
      hdr[9 + a] = gs[a] > 0.f ? (ghi[a] - glo[a]) / (float)CG_GRID : 0.f;
    }
    hdr[12] = __uint_as_float(s_bad);
    // sum(count^2) / n is the mean number of points in a point's own cell.
    // The search uses the finest of 32^3, 16^3, 8^3 whose mean is at least
    // CG_OCC (sparse clouds get coarser cells, so a query's 3x3x3
    // neighbourhood usually holds its nearest point).  A grid whose finest
    // mean exceeds max(256, n / 32) is degenerate: the dense kernels are
    // cheaper.  The sums are added in a fixed order, so the choices are
    // deterministic.
    float sq[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      sq[k] = 0.f;
      for (int v2 = 0; v2 < 16; ++v2) sq[k] += s_sq[k][v2];
    }
    const float nn = (float)n;
    const uint32_t level = sq[0] >= CG_OCC * nn ? 0u : (sq[1] >= CG_OCC * nn ? 1u : 2u);
    hdr[13] = __uint_as_float(n > 0 && sq[0] > occ_lim ? 1u : 0u);
    hdr[14] = __uint_as_float(level);
    hdr[15] = __uint_as_float(trim);
  }
}

// A lane walks cells one by one; a box of more cells than about nr / 64
// costs more to walk than the whole cloud costs the wave to scan together,
// so such lanes (and lanes with no point in their cell's 3x3x3
// neighbourhood) are answered by a wave-wide scan instead.
constexpr int CG_BOX_MIN = 128;  // cells a lane may always walk
__host__ __device__ inline int cg_box_max(int nr) { return max(CG_BOX_MIN, nr >> 6); }

template <typename T, int WG>
__global__ __launch_bounds__(WG, 8) void chamfer_grid_search_kernel(
    const T* __restrict__ xyz1, const T* __restrict__ xyz2, int B, int N, int M, int nqb1,
    int nqb2, const char* __restrict__ ws, CgLayout L, T* __restrict__ dist1,
    T* __restrict__ dist2, int32_t* __restrict__ idx1, int32_t* __restrict__ idx2) {
  using Mg = CgMargin<T>;
  static_assert(WG == 64 * CH_WAVES, "a search workgroup is one 256-query dense block");
  // LDS: the dense block's arrays (degenerate grids only)
  __shared__ __align__(16) char s_mem[sizeof(float4) * CH_WAVES * 64 +
                                      (sizeof(T) + sizeof(int)) * CH_WAVES * WG];
  const int bid = xcd_logical_block(blockIdx.x, gridDim.x);
  int lb = bid;
  const int g1 = B * nqb1;
  const int dir = lb >= g1;
  if (dir) lb -= g1;
  const int nqb = dir ? nqb2 : nqb1;
  const int b = lb / nqb;
  const int qb = lb - b * nqb;
  const int nq = dir ? M : N;
  const int nr = dir ? N : M;
  const int cq = dir, cr = 1 - dir;  // query / reference cloud
  const int64_t PN = cg_pad(N), PM = cg_pad(M);
  const int64_t base_q = (int64_t)b * (PN + PM) + (cq ? PN : 0);
  const int64_t base_r = (int64_t)b * (PN + PM) + (cr ? PN : 0);
  const float4* __restrict__ qs = reinterpret_cast<const float4*>(ws + L.pts) + base_q;
  const float4* __restrict__ rs = reinterpret_cast<const float4*>(ws + L.pts) + base_r;
  const int32_t* __restrict__ cstart =
      reinterpret_cast<const int32_t*>(ws + L.cstart) + (size_t)(2 * b + cr) * CG_CSTRIDE;
  const float* __restrict__ h = reinterpret_cast<const float*>(ws + L.hdr) + (2 * b + cr) * 16;
  const T* __restrict__ rp = (dir ? xyz1 : xyz2) + (size_t)b * nr * 3;  // original order
  const T* __restrict__ qp = (dir ? xyz2 : xyz1) + (size_t)b * nq * 3;
  T* __restrict__ dout = (dir ? dist2 : dist1) + (size_t)b * nq;
  int32_t* __restrict__ iout = (dir ? idx2 : idx1) + (size_t)b * nq;
  int32_t* __restrict__ stats = reinterpret_cast<int32_t*>(const_cast<char*>(ws) + L.stats);

  const int lane = lane_id(), w = wave_id();
  if (__float_as_uint(h[13]) != 0u) {
    // a degenerate reference grid: this workgroup's 256 queries (in original
    // order) are answered by the dense block (every pair evaluated)
    auto& s_ref = *reinterpret_cast<float4(*)[CH_WAVES][64]>(s_mem);
    char* tail = s_mem + sizeof(float4) * CH_WAVES * 64;
    if constexpr (sizeof(T) == 4) {  // two 128-query blocks (keeps the registers low)
      auto& s_d = *reinterpret_cast<T(*)[CH_WAVES][128]>(tail);
      auto& s_i = *reinterpret_cast<int(*)[CH_WAVES][128]>(tail + sizeof(T) * CH_WAVES * 128);
      for (int k = 0; k < WG / 128; ++k)
        chamfer_filter_block<2, CH_FTILE>(qp, rp, nq, nr, qb * (WG / 128) + k, dout, iout, s_ref,
                                          s_d, s_i);
    } else {  // four 64-query blocks (keeps the kernel's registers low)
      auto& s_d = *reinterpret_cast<T(*)[CH_WAVES][64]>(tail);
      auto& s_i = *reinterpret_cast<int(*)[CH_WAVES][64]>(tail + sizeof(T) * CH_WAVES * 64);
      for (int k = 0; k < WG / 64; ++k)
        chamfer_dense_block<T, 1>(qp, rp, nq, nr, qb * (WG / 64) + k, dout, iout, s_d, s_i);
    }
    const int64_t nv = max(0, min(nq - (qb * WG + w * 64), 64));
    if (lane == 0) stats[(size_t)bid * (WG / 64) + w] = (int32_t)min(nv * nr, (int64_t)0x7fffffff);
    return;
  }
  const int pos = qb * WG + (int)threadIdx.x;
  const bool valid = pos < nq;
  const float4 q = qs[min(pos, nq - 1)];
  const int oq = __float_as_int(q.w);
  const bool rbad = __float_as_uint(h[12]) != 0u;
  const bool qbad = max(abs_bits(q.x), max(abs_bits(q.y), abs_bits(q.z))) >= CH_BIG;
  const bool fallback = valid && (rbad || qbad);
  bool far = false;  // answered by the wave-wide scan below
  int examined = 0;
  const unsigned long long kInit = ((unsigned long long)0x7f800000u << 32) | 0x7fffffffu;

  if (valid && !fallback) {
    // grid geometry at the search resolution: G cells per axis, cell
    // (cx, cy, cz) holding the sorted points [cstart[code << 3 lv],
    // cstart[(code + 1) << 3 lv]) -- a Morton-ordered 32^3 cell c lies in
    // the coarser cell c >> 3 lv, and the coarser cell index equals
    // floor((p - lo) * gs / 2^lv) exactly (scaling by a power of two
    // commutes with rounding), so the two views agree
    const int lv = (int)__float_as_uint(h[14]);
    const uint32_t cut = __float_as_uint(h[15]);
    const int G = CG_GRID >> lv, sh = 3 * lv;
    float glo[3], ghi[3], gs[3], cs[3], eps[3];
    const float qv[3] = {q.x, q.y, q.z};
    int ci[3], ga[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      glo[a] = h[a];
      ghi[a] = h[3 + a];
      gs[a] = __builtin_ldexpf(h[6 + a], -lv);
      cs[a] = __builtin_ldexpf(h[9 + a], lv);
      ga[a] = gs[a] > 0.f ? G : 1;
      ci[a] = gs[a] > 0.f ? cg_axis_cell(qv[a], glo[a], gs[a], G) : 0;
      eps[a] = 0x1p-20f * (__builtin_fabsf(glo[a]) + (ghi[a] - glo[a])) + 0x1p-126f;
    }
    // distance from the query to cell c's slab along axis a (a lower bound,
    // widened by the margins); the first / last cell is unbounded on a cut side
    auto axis_gap = [&](int a, int c) {
      const float clo = (cut >> a) & 1u && c == 0
                            ? -__builtin_inff()
                            : (ga[a] > 1 ? glo[a] + (float)c * cs[a] : glo[a]) - eps[a];
      const float chi = (cut >> (3 + a)) & 1u && c == ga[a] - 1
                            ? __builtin_inff()
                            : (ga[a] > 1 ? glo[a] + (float)(c + 1) * cs[a] : ghi[a]) + eps[a];
      return fmaxf(fmaxf(clo - qv[a], qv[a] - chi), 0.f);
    };
    // best (distance, index) as one key: distances here are finite and >= 0,
    // so their bits order like the values, and the index breaks ties
    unsigned long long bkey = kInit;
    auto bdist = [&]() { return __uint_as_float((uint32_t)(bkey >> 32)); };
    const char* __restrict__ rsb = reinterpret_cast<const char*>(rs);
    // evaluate every point of sorted positions [j0, j1)
    auto scan = [&](int j0, int j1) {
      for (int j = j0; j < j1; j += CG_UNROLL) {
        // CG_UNROLL loads in flight; positions past the cell repeat its last
        // point, whose second evaluation cannot change the result
        float4 p[CG_UNROLL];
#pragma unroll
        for (int u = 0; u < CG_UNROLL; ++u)
          p[u] = *reinterpret_cast<const float4*>(rsb + (uint32_t)min(j + u, j1 - 1) * 16u);
#pragma unroll
        for (int u = 0; u < CG_UNROLL; ++u) {
          const float d = cg_dist<T>(p[u], q);
          const unsigned long long key =
              ((unsigned long long)__float_as_uint(d) << 32) | __float_as_uint(p[u].w);
          bkey = key < bkey ? key : bkey;
        }
      }
      examined += j1 - j0;
    };
    auto scan_cell = [&](uint32_t code) { scan(cstart[code << sh], cstart[(code + 1) << sh]); };
    // evaluate every point of cell cc unless its box is farther than the best
    auto visit = [&](int cx, int cy, int cz) {
      const int cc[3] = {cx, cy, cz};
      float gap[3];
#pragma unroll
      for (int a = 0; a < 3; ++a) gap[a] = axis_gap(a, cc[a]);
      if (sq3(gap[0], gap[1], gap[2]) * Mg::lb - Mg::abs > bdist()) return;
      scan_cell(cg_code(cx, cy, cz));
    };
    // phase 1: the query's cell; if it is empty, ring 1, nearest cells
    // first: the six face neighbours (the nearer face of each axis first),
    // then the 12 edge and 8 corner neighbours, each group skipped whole
    // when a lower bound of its cells' gaps (the same per-axis gaps visit
    // computes, combined monotonically) already exceeds the best distance.
    // Nothing within ring 1: the wave-wide scan answers the query.
    visit(ci[0], ci[1], ci[2]);
    int rdone = 0;
    if (bdist() == Lim<float>::inf()) {
      float gn[3];
      int sn[3];
#pragma unroll
      for (int a = 0; a < 3; ++a) {
        // gap to the neighbour below (its upper bound) and above (its lower bound)
        const float gm = ci[a] > 0 ? fmaxf(qv[a] - (glo[a] + (float)ci[a] * cs[a] + eps[a]), 0.f)
                                   : __builtin_inff();
        const float gp = ci[a] < ga[a] - 1
                             ? fmaxf((glo[a] + (float)(ci[a] + 1) * cs[a] - eps[a]) - qv[a], 0.f)
                             : __builtin_inff();
        sn[a] = gm <= gp ? -1 : 1;
        gn[a] = fminf(gm, gp);
      }
      auto inb = [&](int a, int d) { return ci[a] + d >= 0 && ci[a] + d < ga[a]; };
      auto cell = [&](int dx, int dy, int dz) {
        if (inb(0, dx) && inb(1, dy) && inb(2, dz)) visit(ci[0] + dx, ci[1] + dy, ci[2] + dz);
      };
      cell(sn[0], 0, 0);
      cell(0, sn[1], 0);
      cell(0, 0, sn[2]);
      cell(-sn[0], 0, 0);
      cell(0, -sn[1], 0);
      cell(0, 0, -sn[2]);
      const float ge = fminf(fminf(sq3(gn[0], gn[1], 0.f), sq3(gn[0], 0.f, gn[2])),
                             sq3(0.f, gn[1], gn[2]));
      if (!(ge * Mg::lb - Mg::abs > bdist())) {
        for (int e = 0; e < 12; ++e) {  // (a, b) axis pair with signs
          const int pr = e >> 2, sa = (e & 1) ? 1 : -1, sb = (e & 2) ? 1 : -1;
          const int dx = pr == 2 ? 0 : sa, dy = pr == 0 ? sb : (pr == 1 ? 0 : sa);
          const int dz = pr == 0 ? 0 : sb;
          cell(dx, dy, dz);
        }
        if (!(sq3(gn[0], gn[1], gn[2]) * Mg::lb - Mg::abs > bdist()))
          for (int c = 0; c < 8; ++c)
            cell((c & 1) ? 1 : -1, (c & 2) ? 1 : -1, (c & 4) ? 1 : -1);
      }
      rdone = 1;
      far = bdist() == Lim<float>::inf();
    }
    // phase 2: the box of cells within the best distance (cell assignment is
    // monotone in each coordinate, so the box holds every point within it);
    // cells of the rings already walked are skipped.  The gap to a cell is
    // accumulated per axis as the loops descend, so a slab or row whose
    // partial lower bound already exceeds the best distance is skipped whole
    // (the bound only grows with more axes; any summation order rounds by a
    // few u, well inside the 2^-20 margin).  A box of more than
    // cg_box_max(nr) cells goes to the wave-wide scan.
    int blo[3], bhi[3];
    const float bd = bdist();
    const float rad = __builtin_sqrtf((bd + Mg::abs) * Mg::inv) * (1.f + 0x1p-19f);
    int cells = 1;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      const float ra = rad + eps[a] + 0x1p-20f * __builtin_fabsf(qv[a]);
      blo[a] = ga[a] > 1 ? cg_axis_cell(qv[a] - ra, glo[a], gs[a], G) : 0;
      bhi[a] = ga[a] > 1 ? cg_axis_cell(qv[a] + ra, glo[a], gs[a], G) : 0;
      cells *= bhi[a] - blo[a] + 1;
    }
    far = far || cells > cg_box_max(nr);
    if (!far) {
      auto gap2 = [&](int a, int c) {
        const float g = axis_gap(a, c);
        return g * g;
      };
      for (int cz = blo[2]; cz <= bhi[2]; ++cz) {
        const float gz = gap2(2, cz);
        if (gz * Mg::lb - Mg::abs > bdist()) continue;
        const uint32_t kz = cg_spread((uint32_t)cz) << 2;
        const int dz = abs(cz - ci[2]);
        for (int cy = blo[1]; cy <= bhi[1]; ++cy) {
          const float gzy = gz + gap2(1, cy);
          if (gzy * Mg::lb - Mg::abs > bdist()) continue;
          const uint32_t kzy = kz | (cg_spread((uint32_t)cy) << 1);
          const int dzy = max(dz, abs(cy - ci[1]));
          for (int cx = blo[0]; cx <= bhi[0]; ++cx) {
            if (max(dzy, abs(cx - ci[0])) <= rdone) continue;
            if ((gzy + gap2(0, cx)) * Mg::lb - Mg::abs > bdist()) continue;
            scan_cell(kzy | cg_spread((uint32_t)cx));
          }
        }
      }
      dout[oq] = (T)bdist();
      iout[oq] = (int)(uint32_t)bkey;
    }
  }
  // far queries: the wave scans every reference point (sorted order, same
  // key), one query at a time
  for (uint64_t fm = __ballot(far); fm; fm &= fm - 1) {
    const int l = __builtin_ctzll(fm);
    const float4 ql = make_float4(__shfl(q.x, l), __shfl(q.y, l), __shfl(q.z, l), 0.f);
    unsigned long long k = kInit;
    for (int j = lane; j < nr; j += 64) {
      const float4 p = rs[j];
      const unsigned long long key =
          ((unsigned long long)__float_as_uint(cg_dist<T>(p, ql)) << 32) | __float_as_uint(p.w);
      k = key < k ? key : k;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const unsigned long long x = __shfl_xor(k, o);
      k = x < k ? x : k;
    }
    if (lane == l) {
      dout[oq] = (T)__uint_as_float((uint32_t)(k >> 32));
      iout[oq] = (int)(uint32_t)k;
    }
    examined += lane == 0 ? nr : 0;
  }
  {  // points evaluated by this wave
    int e = examined;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) e += __shfl_xor(e, o);
    if (lane == 0) stats[(size_t)bid * (WG / 64) + w] = e;
  }
  // queries that need the reference's full rule: the wave scans one at a time
  uint64_t fb = __ballot(fallback);
  while (fb) {
    const int l = __builtin_ctzll(fb);
    fb &= fb - 1;
    const int o = __shfl(oq, l);
    T md;
    int mi;
    chunk_scan(qp[3 * o], qp[3 * o + 1], qp[3 * o + 2], rp, 0, nr, lane, md, mi);
    if (mi == 0x7fffffff) {  // no reference counts: cannot happen with nr > 0
      md = (T)0;
      mi = 0;
    }
    if (lane == 0) {
      dout[o] = md;
      iout[o] = mi;
    }
  }
}

__global__ __launch_bounds__(256) void chamfer_stats_kernel(const int32_t* __restrict__ stats,
                                                            int64_t n, int64_t* __restrict__ out) {
  __shared__ int64_t part[4];
  int64_t s = 0;
  for (int64_t k = threadIdx.x; k < n; k += 256) s += stats[k];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) out[0] = part[0] + part[1] + part[2] + part[3];
}

int64_t chamfer_prune_workspace(int64_t B, int64_t N, int64_t M) {
  return cg_layout(B, N, M).total;
}

template <typename T>
static void launch_prune(const void* x1, const void* x2, int B, int N, int M, void* d1, void* d2,
                         int32_t* i1, int32_t* i2, void* ws, hipStream_t s, uint32_t* zero) {
  const CgLayout L = cg_layout(B, N, M);
  if (std::max(N, M) <= 1024 * 8)
    hipLaunchKernelGGL((chamfer_grid_sort_kernel<T, 8>), dim3(2 * B), dim3(1024), 0, s,
                       (const T*)x1, (const T*)x2, N, M, (char*)ws, L, zero);
  else
    hipLaunchKernelGGL((chamfer_grid_sort_kernel<T, 0>), dim3(2 * B), dim3(1024), 0, s,
                       (const T*)x1, (const T*)x2, N, M, (char*)ws, L, zero);
  const int nqb1 = (N + CG_WG - 1) / CG_WG, nqb2 = (M + CG_WG - 1) / CG_WG;
  hipLaunchKernelGGL((chamfer_grid_search_kernel<T, CG_WG>), dim3(B * (nqb1 + nqb2)),
                     dim3(CG_WG), 0, s, (const T*)x1, (const T*)x2, B, N, M, nqb1, nqb2,
                     (const char*)ws, L, (T*)d1, (T*)d2, i1, i2);
}

void launch_chamfer_fwd_prune(int dtype, const void* x1, const void* x2, int B, int N, int M,
                              void* d1, void* d2, int32_t* i1, int32_t* i2, void* ws,
                              hipStream_t s, uint32_t* zero) {
  if (dtype == TPO_F16)
    launch_prune<half_t>(x1, x2, B, N, M, d1, d2, i1, i2, ws, s, zero);
  else
    launch_prune<float>(x1, x2, B, N, M, d1, d2, i1, i2, ws, s, zero);
}

void launch_chamfer_prune_stats(const void* ws, int64_t B, int64_t N, int64_t M, int64_t* out,
                                hipStream_t s) {
  const CgLayout L = cg_layout(B, N, M);
  hipLaunchKernelGGL(chamfer_stats_kernel, dim3(1), dim3(256), 0, s,
                     reinterpret_cast<const int32_t*>((const char*)ws + L.stats),
                     cg_grid_size(B, N, M) * (CG_WG / 64), out);
}

}  // namespace tpo
