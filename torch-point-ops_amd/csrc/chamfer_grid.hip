// chamfer_grid.hip -- Chamfer forward for float and half clouds by exact grid
// search (replaces chamfer_dist_kernel, chamfer.cu:36-167, when the caller
// provides a workspace and both clouds have at least CH_PRUNE_MIN points).
// Half coordinates are held as float copies (exact) for the grid; distances
// are computed in half as the reference does, and the pruning margins cover
// half rounding (CgMargin).
//
// 1. chamfer_grid_sort_kernel, two workgroups per (batch, cloud) for clouds
//    of up to 8192 points (one above): the cloud's bounding box, a counting
//    sort of its points into a 32^3 grid of cells (cells in Morton order, so
//    neighbouring cells are mostly close in memory), the sorted points as
//    (original index, x, y, z) and the start of every cell.  The two
//    workgroups build the same grid and each writes half of it.
// 2. chamfer_grid_search_kernel: one query per lane, queries taken in the
//    sorted (Morton) order of their own cloud so a wave's queries lie close
//    together.  Per query: its own cell; if that is empty, ring 1 (the 26
//    cells around it); then the box of cells that can hold a point within
//    the best distance found (cell assignment is monotone in each
//    coordinate, and the box is widened by 2^-19 relative plus the rounding
//    of its bounds), without the cells scanned before.  A cell is skipped
//    when a lower bound of its squared distance, rounded down by 2^-20
//    relative, exceeds the query's best distance: the reference's float
//    distance of any of its points is then strictly larger (its relative
//    error is <= 5u), so neither a smaller distance nor a tie with a lower
//    index is missed.  Cell boxes are widened by 2^-20 (|lo| + extent) per
//    side, which covers the rounding of the cell assignment.  Every point of
//    a scanned cell is evaluated with the reference formula
//    (chamfer.cu:64-67, same bits), keeping the smallest (distance, original
//    index) -- the reference's first-index rule.
//    The wave shares this work out instead of each lane walking its own
//    cells: every lane contributes segments of items (its box's cells; a
//    scanned cell's points), and the wave takes the items in order, 64 R
//    a round (R consecutive items to a lane), each lane finding the segment
//    of its items from the marked segment starts and a running maximum over
//    the lanes (DPP).  Lanes stay busy however unevenly the queries' work is
//    spread.  Each query's best key sits in LDS and takes the items' results
//    by 64-bit LDS atomicMin (one per run of a lane's items of one query).
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
// scans coarse 8^3 cells nearest first while a cell can hold a nearer point.
// Results are identical to
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
constexpr int CG_OCC = 2;     // mean own-cell occupancy the search resolution aims at

__host__ __device__ inline int64_t cg_pad(int64_t n) { return (n + 63) & ~(int64_t)63; }

// Byte offsets of the workspace regions (all 256-byte aligned).
struct CgLayout {
  int64_t hdr;     // 2B x 16 floats: lo[3], hi[3], cells per unit[3], cell size[3] (32^3),
                   // bad, degenerate, level (search cells are 2^level of them per axis),
                   // cut sides (bit a: axis a cut below, 3 + a: above; the boundary
                   // cells on a cut side are unbounded)
  int64_t pts;     // float4 per padded point: sorted (original index bits, x, y, z)
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

// (fmaxf returns its non-NaN operand, so a NaN position lands in cell 0)
__device__ __forceinline__ int cg_axis_cell(float p, float lo, float sc, int g = CG_GRID) {
  return (int)fminf(fmaxf((p - lo) * sc, 0.f), (float)(g - 1));
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
  return sq3((float)(p.y - q.y), (float)(p.z - q.z), (float)(p.w - q.w));
}
template <>
__device__ __forceinline__ float cg_dist<half_t>(const float4& p, const float4& q) {
  return (float)sq3((half_t)((half_t)p.y - (half_t)q.y), (half_t)((half_t)p.z - (half_t)q.z),
                    (half_t)((half_t)p.w - (half_t)q.w));
}

// The same distance with the query as three coordinates.
template <typename T>
__device__ __forceinline__ float cg_dist3(const float4& p, float qx, float qy, float qz);
template <>
__device__ __forceinline__ float cg_dist3<float>(const float4& p, float qx, float qy, float qz) {
  return sq3((float)(p.y - qx), (float)(p.z - qy), (float)(p.w - qz));
}
template <>
__device__ __forceinline__ float cg_dist3<half_t>(const float4& p, float qx, float qy, float qz) {
  return (float)sq3((half_t)((half_t)p.y - (half_t)qx), (half_t)((half_t)p.z - (half_t)qy),
                    (half_t)((half_t)p.w - (half_t)qz));
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

// Wave reductions of the sort by DPP steps whose result reaches lane 63:
// pairs, quads, 8 (half-row mirror), 16 (row mirror: after these four every
// lane holds its row's result), then rows 0-1 and 2-3 (row_bcast:15) and all
// four (row_bcast:31).  A lane that a step does not write keeps its value.
template <int CTRL, int RM>
__device__ __forceinline__ uint32_t cg_dpp_keep(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, RM, 0xf, false);
}
template <typename F>
__device__ __forceinline__ uint32_t cg_row_reduce(uint32_t v, F&& op) {
  v = op(v, cg_dpp_keep<0xB1, 0xf>(v));   // quad_perm [1,0,3,2]
  v = op(v, cg_dpp_keep<0x4E, 0xf>(v));   // quad_perm [2,3,0,1]
  v = op(v, cg_dpp_keep<0x141, 0xf>(v));  // row_half_mirror
  v = op(v, cg_dpp_keep<0x140, 0xf>(v));  // row_mirror
  return v;
}
template <typename F>
__device__ __forceinline__ uint32_t cg_wave_reduce63(uint32_t v, F&& op) {
  v = cg_row_reduce(v, op);
  v = op(v, cg_dpp_keep<0x142, 0xa>(v));  // row_bcast:15 into rows 1, 3
  v = op(v, cg_dpp_keep<0x143, 0xc>(v));  // row_bcast:31 into rows 2, 3
  return v;
}
// fminf / fmaxf on float bits (NaN ignored, as those functions do)
struct CgFmin {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const {
    return __float_as_uint(fminf(__uint_as_float(a), __uint_as_float(b)));
  }
};
struct CgFmax {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }
};
struct CgAdd {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a + b; }
};
struct CgMaxU {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; }
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
  // PPT > 0: two workgroups per cloud; both build the same grid (box,
  // histogram, scan) and each writes half of it: the cell starts and the
  // sorted points of cells [hf, hf + 1) * CG_CELLS / 2
  constexpr int HALVES = PPT > 0 ? 2 : 1;
  int b = blockIdx.x / (2 * HALVES), j = blockIdx.x % (2 * HALVES);
  batch_home_block(blockIdx.x, gridDim.x / (2 * HALVES), 2 * HALVES, b, j);
  const int c = j / HALVES, hf = j % HALVES;  // cloud, half
  const int cl = 2 * b + c;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int n = c ? M : N;
  if (zero && blockIdx.x == 0 && tid == 0) *zero = 0u;
  const int64_t PN = cg_pad(N), PM = cg_pad(M);
  const int64_t base = (int64_t)b * (PN + PM) + (c ? PN : 0);
  const TI* __restrict__ P = (c ? xyz2 : xyz1) + (size_t)b * n * 3;
  float* __restrict__ hdr = reinterpret_cast<float*>(ws + L.hdr) + (size_t)cl * 16;
  float4* __restrict__ pts = reinterpret_cast<float4*>(ws + L.pts) + base;
  int32_t* __restrict__ cstart =
      reinterpret_cast<int32_t*>(ws + L.cstart) + (size_t)cl * CG_CSTRIDE;
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
  for (int a = 0; a < 3; ++a) {
    lo[a] = __uint_as_float(cg_wave_reduce63(__float_as_uint(lo[a]), CgFmin{}));
    hi[a] = __uint_as_float(cg_wave_reduce63(__float_as_uint(hi[a]), CgFmax{}));
  }
  if (lane == 63)
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
    // the 16 waves' values, one a lane of each row, reduced within the row
    float x = __uint_as_float(cg_row_reduce(__float_as_uint(red[a][lane & 15]), CgFmin{}));
    float z = __uint_as_float(cg_row_reduce(__float_as_uint(red[3 + a][lane & 15]), CgFmax{}));
    x = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
    z = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(z)));
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
    if constexpr (PPT > 0) {
      // all of a thread's atomics are issued before any returned rank is
      // used, so their LDS round trips overlap; a slot past the cloud (a copy
      // of the last point) adds 0
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        hx[i] = (uint32_t)cg_hidx(code_of(px[i], py[i], pz[i]));
        rk[i] = atomicAdd(&cnt[hx[i]], tid + 1024 * i < n ? 1u : 0u);
      }
#pragma unroll
      for (int i = 0; i < PPT; ++i)
        if (tid + 1024 * i < n) mr = max(mr, rk[i] + 1);
    } else {
      for (int i = 0; i < iters; ++i) {
        const int k = tid + 1024 * i;
        if (k >= n) break;
        float x, y, z;
        point(i, k, x, y, z);
        const uint32_t r = atomicAdd(&cnt[cg_hidx(code_of(x, y, z))], 1u);
        mr = max(mr, r + 1);
        rank[k] = (int32_t)r;
      }
    }
    mr = cg_wave_reduce63(mr, CgMaxU{});
    if (lane == 63) atomicMax(&s_maxc, mr);
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
      // and its neighbour's an 8^3 cell), reduced in a fixed order; with the
      // points in registers (n <= 8192) in integers, every sum below 2^26
      if constexpr (PPT > 0) {
        uint32_t q0 = 0, q1 = 0;
#pragma unroll
        for (int i = 0; i < CPT; i += 8) {
          uint32_t c8 = 0;
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            q0 += v[i + k] * v[i + k];
            c8 += v[i + k];
          }
          q1 += c8 * c8;
        }
        const uint32_t c64 = sum + cg_dpp_keep<0xB1, 0xf>(sum);  // this thread's and its pair's
        uint32_t q2 = (lane & 1) ? 0u : c64 * c64;
        q0 = cg_wave_reduce63(q0, CgAdd{});
        q1 = cg_wave_reduce63(q1, CgAdd{});
        q2 = cg_wave_reduce63(q2, CgAdd{});
        if (lane == 63) {
          s_sq[0][w] = (float)q0;
          s_sq[1][w] = (float)q1;
          s_sq[2][w] = (float)q2;
        }
      } else {
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
  for (int k = tid + hf * (CG_CELLS / 4 / HALVES); k < (hf + 1) * (CG_CELLS / 4 / HALVES);
       k += 1024) {  // coalesced, 4 cells per store
    const int c0 = cg_hidx(4 * k);  // the 4 cells share one padded run of 32
    reinterpret_cast<int4*>(cstart)[k] =
        make_int4((int)cnt[c0], (int)cnt[c0 + 1], (int)cnt[c0 + 2], (int)cnt[c0 + 3]);
  }
  if constexpr (PPT > 0) {
    // sorted positions into registers; once every read of the counts is done
    // the points are placed in LDS and written out in order, coalesced
    // this half's sorted positions [p0, p1)
    const uint32_t p0 = cnt[cg_hidx(hf * (CG_CELLS / 2))];
    const uint32_t p1 = hf ? (uint32_t)n : cnt[cg_hidx(CG_CELLS / 2)];
    uint32_t at[R];
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int k = tid + 1024 * i;
      at[i] = k < n ? cnt[hx[i]] + rk[i] : 0xffffffffu;
    }
    __syncthreads();
    float4* __restrict__ stage = reinterpret_cast<float4*>(cnt);
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int k = tid + 1024 * i;
      if (at[i] >= p0 && at[i] < p1)
        stage[at[i] - p0] = make_float4(__int_as_float(k), px[i], py[i], pz[i]);
    }
    __syncthreads();
    for (uint32_t pos = p0 + tid; pos < p1; pos += 1024) pts[pos] = stage[pos - p0];
    if (hf == HALVES - 1)
      for (int pos = n + tid; pos < cg_pad(n); pos += 1024)
        pts[pos] = make_float4(__int_as_float(-1), 0.f, 0.f, 0.f);
  } else {
    for (int i = 0; i < iters; ++i) {
      const int k = tid + 1024 * i;
      if (k >= n) break;
      float x, y, z;
      point(i, k, x, y, z);
      pts[cnt[cg_hidx(code_of(x, y, z))] + (uint32_t)rank[k]] =
          make_float4(__int_as_float(k), x, y, z);
    }
    for (int pos = n + tid; pos < cg_pad(n); pos += 1024)
      pts[pos] = make_float4(__int_as_float(-1), 0.f, 0.f, 0.f);
  }
  if (tid == 0 && hf == 0) {
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

// A query whose box holds more cells than about nr / 64 would cost the wave
// more than a scan of the whole cloud together, so such queries (and those
// with no point in their cell's 3x3x3 neighbourhood) are answered by a
// wave-wide scan instead.
constexpr int CG_BOX_MIN = 128;  // cells a box may always hold
// a search wave's LDS rows
constexpr int CG_R = 4;   // points a lane evaluates per round of the search
constexpr int CG_RC = 2;  // cells a lane tests per round of a walk
struct CgWaveLds {
  unsigned long long key[64];
  float4 q[64];
  int4 box[64];
  int2 seg[64 * CG_RC];  // per segment: first sorted position - first item, query lane
  int mark[64 * CG_R];
};
__host__ __device__ inline int cg_box_max(int nr) { return max(CG_BOX_MIN, nr >> 6); }

// Wave-level pieces of the search (every lane of the wave active).
__device__ __forceinline__ void cg_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
template <int CTRL, int ROWMASK>
__device__ __forceinline__ int cg_dpp(int v) {  // lanes without a source read 0
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWMASK, 0xf, true);
}
// inclusive prefix sum / maximum (of values >= 0) over the lanes: row_shr 1, 2,
// 4, 8 within rows of 16, then row_bcast:15 into rows 1, 3 and row_bcast:31
// into rows 2, 3
__device__ __forceinline__ int cg_scan_add(int v) {
  v += cg_dpp<0x111, 0xf>(v);
  v += cg_dpp<0x112, 0xf>(v);
  v += cg_dpp<0x114, 0xf>(v);
  v += cg_dpp<0x118, 0xf>(v);
  v += cg_dpp<0x142, 0xa>(v);
  v += cg_dpp<0x143, 0xc>(v);
  return v;
}
__device__ __forceinline__ int cg_scan_max(int v) {
  v = max(v, cg_dpp<0x111, 0xf>(v));
  v = max(v, cg_dpp<0x112, 0xf>(v));
  v = max(v, cg_dpp<0x114, 0xf>(v));
  v = max(v, cg_dpp<0x118, 0xf>(v));
  v = max(v, cg_dpp<0x142, 0xa>(v));
  v = max(v, cg_dpp<0x143, 0xc>(v));
  return v;
}
// Every lane holds RC segments of len[v] >= 0 items (segment RC lane + v);
// the wave hands the items out in order, 64 R a round, R consecutive ones to
// a lane: body(ok, s, i) runs on every lane each round, with item i[u]
// (ok[u]: it exists) of segment s[u], u < R (s is non-decreasing in u and
// over the lanes).  The segment of each item comes from the segment starts
// marked in the wave's LDS row mark (64 R ints) and a running maximum over
// the items.
template <int R, int RC, typename F>
__device__ __forceinline__ void cg_flat(const int (&len)[RC], int* __restrict__ mark, F&& body) {
  const int lane = lane_id();
  int tot = 0;
#pragma unroll
  for (int v = 0; v < RC; ++v) tot += len[v];
  const int incl = cg_scan_add(tot);
  const int total = __builtin_amdgcn_readlane(incl, 63);
  int ex[RC];  // first item of each segment
#pragma unroll
  for (int v = 0; v < RC; ++v) ex[v] = v ? ex[v - 1] + len[v - 1] : incl - tot;
  int carry = 0;  // 1 + the segment holding the previous round's last item
  for (int base = 0; base < total; base += 64 * R) {
    if constexpr (R == 4) {
      reinterpret_cast<int4*>(mark)[lane] = make_int4(0, 0, 0, 0);
    } else {
#pragma unroll
      for (int u = 0; u < R; ++u) mark[R * lane + u] = 0;
    }
    cg_wave_sync();
#pragma unroll
    for (int v = 0; v < RC; ++v)
      if (len[v] > 0 && ex[v] >= base && ex[v] < base + 64 * R) mark[ex[v] - base] = RC * lane + v + 1;
    cg_wave_sync();
    int lm[R];
    if constexpr (R == 4) {
      const int4 m4 = reinterpret_cast<const int4*>(mark)[lane];
      lm[0] = m4.x;
      lm[1] = max(m4.x, m4.y);
      lm[2] = max(lm[1], m4.z);
      lm[3] = max(lm[2], m4.w);
    } else {
#pragma unroll
      for (int u = 0; u < R; ++u) lm[u] = u ? max(lm[u - 1], mark[R * lane + u]) : mark[R * lane];
    }
    const int inc = cg_scan_max(lm[R - 1]);
    // the maximum over the lanes before this one (DPP wave_shr:1, lane 0 reads 0)
    const int c0 = max(carry, __builtin_amdgcn_update_dpp(0, inc, 0x138, 0xf, 0xf, true));
    carry = max(carry, __builtin_amdgcn_readlane(inc, 63));
    int sg[R], it[R];
    bool ok[R];
#pragma unroll
    for (int u = 0; u < R; ++u) {
      sg[u] = max(max(c0, lm[u]) - 1, 0);
      it[u] = base + R * lane + u;
      ok[u] = it[u] < total;
    }
    body(ok, sg, it);
    cg_wave_sync();
  }
}

template <typename T, int WG>
__global__ __launch_bounds__(WG, 8) void chamfer_grid_search_kernel(
    const T* __restrict__ xyz1, const T* __restrict__ xyz2, int B, int N, int M, int nqb1,
    int nqb2, const char* __restrict__ ws, CgLayout L, T* __restrict__ dist1,
    T* __restrict__ dist2, int32_t* __restrict__ idx1, int32_t* __restrict__ idx2) {
  using Mg = CgMargin<T>;
  static_assert(WG == 64 * CH_WAVES, "a search workgroup is one 256-query dense block");
  // LDS: the dense block's arrays (degenerate grids only) or the waves' rows
  constexpr size_t kDense = sizeof(float4) * CH_WAVES * 64 + (sizeof(T) + sizeof(int)) * CH_WAVES * WG;
  __shared__ __align__(16) char s_mem[kDense > sizeof(CgWaveLds) * CH_WAVES ? kDense
                                                                           : sizeof(CgWaveLds) * CH_WAVES];
  const int bid = xcd_logical_block(blockIdx.x, gridDim.x);
  int b, qb, dir;
  {
    int j;
    if (batch_home_block(blockIdx.x, B, nqb1 + nqb2, b, j)) {
      dir = j >= nqb1;
      qb = dir ? j - nqb1 : j;
    } else {
      int lb = bid;
      const int g1 = B * nqb1;
      dir = lb >= g1;
      if (dir) lb -= g1;
      const int nqb = dir ? nqb2 : nqb1;
      b = __builtin_amdgcn_readfirstlane(lb / nqb);  // uniform: scalar loads below
      qb = lb - b * nqb;
    }
  }
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
  const bool rbad = __float_as_uint(h[12]) != 0u;
  const bool qbad = max(abs_bits(q.y), max(abs_bits(q.z), abs_bits(q.w))) >= CH_BIG;
  const bool fallback = valid && (rbad || qbad);
  const bool act = valid && !fallback;  // answered by the grid search
  int examined = 0;  // points the wave evaluated (wave-uniform)
  const unsigned long long kInit = ((unsigned long long)0x7f800000u << 32) | 0x7fffffffu;

  // grid geometry at the search resolution: G cells per axis, cell
  // (cx, cy, cz) holding the sorted points [cstart[code << 3 lv],
  // cstart[(code + 1) << 3 lv]) -- a Morton-ordered 32^3 cell c lies in
  // the coarser cell c >> 3 lv, and the coarser cell index equals
  // floor((p - lo) * gs / 2^lv) exactly (scaling by a power of two
  // commutes with rounding), so the two views agree
  // (wave-uniform values, pinned to SGPRs)
  auto U = [](float x) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x))); };
  const int lv = __builtin_amdgcn_readfirstlane((int)__float_as_uint(h[14]));
  const uint32_t cut = (uint32_t)__builtin_amdgcn_readfirstlane((int)__float_as_uint(h[15]));
  const int G = CG_GRID >> lv, sh = 3 * lv;
  float glo[3], ghi[3], gs[3], cs[3], eps[3];
  const float qv[3] = {q.y, q.z, q.w};
  int ci[3], ga[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    glo[a] = U(h[a]);
    ghi[a] = U(h[3 + a]);
    gs[a] = U(__builtin_ldexpf(h[6 + a], -lv));
    cs[a] = U(__builtin_ldexpf(h[9 + a], lv));
    ga[a] = gs[a] > 0.f ? G : 1;
    ci[a] = gs[a] > 0.f ? cg_axis_cell(qv[a], glo[a], gs[a], G) : 0;
    eps[a] = U(0x1p-20f * (__builtin_fabsf(glo[a]) + (ghi[a] - glo[a])) + 0x1p-126f);
  }
  // distance from coordinate x to cell c's slab along axis a (a lower bound,
  // widened by the margins); the first / last cell is unbounded on a cut side
  auto axis_gap = [&](int a, int c, float x) {
    const float clo = (cut >> a) & 1u && c == 0
                          ? -__builtin_inff()
                          : (ga[a] > 1 ? glo[a] + (float)c * cs[a] : glo[a]) - eps[a];
    const float chi = (cut >> (3 + a)) & 1u && c == ga[a] - 1
                          ? __builtin_inff()
                          : (ga[a] > 1 ? glo[a] + (float)(c + 1) * cs[a] : ghi[a]) + eps[a];
    return fmaxf(fmaxf(clo - x, x - chi), 0.f);
  };

  // the wave's LDS rows: best (distance, index) key per query (distances here
  // are finite and >= 0, so their bits order like the values and the index
  // breaks ties), the queries, the cell boxes being walked, segment marks
  auto& sg = *reinterpret_cast<CgWaveLds(*)[CH_WAVES]>(s_mem);
  unsigned long long* __restrict__ wkey = sg[w].key;
  float4* __restrict__ wq = sg[w].q;
  int4* __restrict__ wbox = sg[w].box;
  int* __restrict__ wmark = sg[w].mark;
  int2* __restrict__ wseg = sg[w].seg;
  wkey[lane] = kInit;
  wq[lane] = make_float4(q.y, q.z, q.w, q.x);  // coordinates first, then the index
  // the query's cell, packed (5 bits an axis); later phases read the query
  // back from wq, which keeps the registers low
  const int cpk = ci[0] | ci[1] << 5 | ci[2] << 10;
  cg_wave_sync();
  auto best = [&](int l) { return __uint_as_float((uint32_t)(wkey[l] >> 32)); };

  // every lane holds cnt sorted points from j0 on, for the query of lane own:
  // the wave evaluates them all, 64 a round, with the reference formula
  // (chamfer.cu:64-67, same bits), keeping each query's smallest key
  auto scan_segs = [&](auto rc, const int (&cnt)[decltype(rc)::value],
                       const int (&j0)[decltype(rc)::value], const int (&own)[decltype(rc)::value]) {
    constexpr int RC = decltype(rc)::value;
    cg_wave_sync();
    {
      int tot = 0;
#pragma unroll
      for (int v = 0; v < RC; ++v) tot += cnt[v];
      const int incl = cg_scan_add(tot);
      examined += __builtin_amdgcn_readlane(incl, 63);  // the wave's points this call
      int e = incl - tot;
#pragma unroll
      for (int v = 0; v < RC; ++v) {
        wseg[RC * lane + v] = make_int2(j0[v] - e, own[v]);
        e += cnt[v];
      }
    }
    cg_flat<CG_R, RC>(cnt, wmark, [&](const bool (&ok)[CG_R], const int (&sn)[CG_R], const int (&it)[CG_R]) {
      float4 p[CG_R];
      int o[CG_R];
      const char* __restrict__ rsb = reinterpret_cast<const char*>(rs);
#pragma unroll
      for (int u = 0; u < CG_R; ++u) {
        // an item past the last one loads a point of the same reference
        // cloud for some query of the wave: a valid candidate, harmless
        const int2 e = wseg[sn[u]];
        p[u] = *reinterpret_cast<const float4*>(rsb + (uint32_t)min(e.x + it[u], nr - 1) * 16u);
        o[u] = e.y;
      }
#pragma unroll
      for (int u = 1; u < CG_R; ++u) o[u] = ok[u] ? o[u] : o[u - 1];
      // the lane's items belong to non-decreasing query lanes: the minimum
      // over each run of one query (branch-free), then one atomic per run
      unsigned long long r[CG_R];
#pragma unroll
      for (int u = 0; u < CG_R; ++u) {
        const float4 qq = wq[o[u]];
        const float d = cg_dist3<T>(p[u], qq.x, qq.y, qq.z);
        const unsigned long long key =
            (unsigned long long)__float_as_uint(d) << 32 | __float_as_uint(p[u].x);
        r[u] = u > 0 && o[u] == o[u - 1] && r[u - 1] < key ? r[u - 1] : key;
      }
#pragma unroll
      for (int u = 0; u + 1 < CG_R; ++u)
        if (o[u + 1] != o[u]) atomicMin(&wkey[o[u]], r[u]);
      atomicMin(&wkey[o[CG_R - 1]], r[CG_R - 1]);
    });
  };
  // every lane holds a box of V cells (its wbox row: lower corner, extents,
  // own cell, skip radius rd): the wave walks all of them, 64 cells a round;
  // a cell within Chebyshev distance rd of its query's cell was scanned
  // before, and a cell whose lower bound of the squared distance, rounded
  // down by 2^-20 relative, exceeds the query's best distance is skipped: the
  // reference's float distance of any of its points is then strictly larger
  // (its relative error is <= 5u), so neither a smaller distance nor a tie
  // with a lower index is missed.  The cells that remain are scanned.
  auto walk = [&](int V) {
    cg_wave_sync();
    const int vex = cg_scan_add(V) - V;  // first item of each box
    const int Vv[1] = {V};
    cg_flat<CG_RC, 1>(Vv, wmark, [&](const bool (&okv)[CG_RC], const int (&sv)[CG_RC], const int (&iv)[CG_RC]) {
      int cnt[CG_RC], j0[CG_RC];
#pragma unroll
      for (int v = 0; v < CG_RC; ++v) {
        const int s = sv[v];
        const int k = iv[v] - __shfl(vex, s);
        cnt[v] = 0;
        j0[v] = 0;
        if (okv[v]) {
          const int4 bx = wbox[s];
          const int nx = (bx.x >> 17) & 63, ny = (bx.x >> 23) & 63;
          // k = (dz * ny + dy) * nx + dx; the float quotients are exact (the
          // reciprocals' error is far below the 1/(2n) margin of k + 1/2)
          const int t = (int)(((float)k + 0.5f) * __int_as_float(bx.z));
          const int dz = (int)(((float)t + 0.5f) * __int_as_float(bx.w));
          const int cx = (bx.x & 31) + (k - t * nx);
          const int cy = ((bx.x >> 5) & 31) + (t - dz * ny);
          const int cz = ((bx.x >> 10) & 31) + dz;
          const int rd = ((bx.x >> 15) & 3) - 1;
          const int cheb = max(abs(cx - (bx.y & 31)),
                               max(abs(cy - ((bx.y >> 5) & 31)), abs(cz - ((bx.y >> 10) & 31))));
          const float4 qq = wq[s];
          const float g2 = sq3(axis_gap(0, cx, qq.x), axis_gap(1, cy, qq.y), axis_gap(2, cz, qq.z));
          if (cheb > rd && !(g2 * Mg::lb - Mg::abs > best(s))) {
            const uint32_t code = cg_code(cx, cy, cz);
            j0[v] = cstart[code << sh];
            cnt[v] = cstart[(code + 1) << sh] - j0[v];
          }
        }
      }
      scan_segs(std::integral_constant<int, CG_RC>{}, cnt, j0, sv);
    });
  };
  auto set_box = [&](const int (&lo)[3], const int (&hi)[3], int rd) {
    const int nx = hi[0] - lo[0] + 1, ny = hi[1] - lo[1] + 1;
    wbox[lane] = make_int4(lo[0] | lo[1] << 5 | lo[2] << 10 | (rd + 1) << 15 | nx << 17 | ny << 23,
                           cpk, __float_as_int(1.f / (float)nx),
                           __float_as_int(1.f / (float)ny));
    return nx * ny * (hi[2] - lo[2] + 1);
  };

  // phase 1: the query's own cell
  {
    const uint32_t code = cg_code(ci[0], ci[1], ci[2]);
    int j0 = 0, cnt = 0;
    if (act) {
      j0 = cstart[code << sh];
      cnt = cstart[(code + 1) << sh] - j0;
    }
    const int c1[1] = {cnt}, j1[1] = {j0}, o1[1] = {lane};
    scan_segs(std::integral_constant<int, 1>{}, c1, j1, o1);
  }
  cg_wave_sync();
  // phase 2: queries whose own cell is empty walk ring 1 (the 26 cells
  // around it); nothing there: the wave-wide scan below answers the query
  const bool ring = act && best(lane) == Lim<float>::inf();
  if (__ballot(ring)) {
    int V = 0;
    if (ring) {
      int lo[3], hi[3];
#pragma unroll
      for (int a = 0; a < 3; ++a) {
        const int c = (cpk >> (5 * a)) & 31;
        lo[a] = max(c - 1, 0);
        hi[a] = min(c + 1, ga[a] - 1);
      }
      V = set_box(lo, hi, 0);
    }
    walk(V);
    cg_wave_sync();
  }
  // phase 3: the box of cells within the best distance (cell assignment is
  // monotone in each coordinate, so the box holds every point within it),
  // without the cells walked before; a box of more than cg_box_max(nr)
  // cells goes to the wave-wide scan
  const float bd = best(lane);
  bool far = act && bd == Lim<float>::inf();
  {
    int V = 0;
    if (act && !far) {
      const float4 qm = wq[lane];
      const float qa[3] = {qm.x, qm.y, qm.z};
      const float rad = __builtin_sqrtf((bd + Mg::abs) * Mg::inv) * (1.f + 0x1p-19f);
      int lo[3], hi[3], cells = 1;
#pragma unroll
      for (int a = 0; a < 3; ++a) {
        const float ra = rad + eps[a] + 0x1p-20f * __builtin_fabsf(qa[a]);
        lo[a] = ga[a] > 1 ? cg_axis_cell(qa[a] - ra, glo[a], gs[a], G) : 0;
        hi[a] = ga[a] > 1 ? cg_axis_cell(qa[a] + ra, glo[a], gs[a], G) : 0;
        cells *= hi[a] - lo[a] + 1;
      }
      far = cells > cg_box_max(nr);
      if (!far) V = set_box(lo, hi, ring ? 1 : 0);
    }
    walk(V);
    cg_wave_sync();
  }
  if (act && !far) {
    const unsigned long long kb = wkey[lane];
    const int o = __float_as_int(wq[lane].w);
    dout[o] = (T)__uint_as_float((uint32_t)(kb >> 32));
    iout[o] = (int)(uint32_t)kb;
  }
  // far queries (nothing in the cell's 3x3x3 neighbourhood, or a box of too
  // many cells): one query at a time over the coarse grid of 8^3 cells
  // (Morton order nests the cells: a coarse cell is the run of its 64 fine
  // 32^3 cells).  Each lane bounds 8 coarse cells from below as the walk
  // bounds cells; the wave scans the open cell with the smallest bound (its
  // run of sorted points, 64 a round, a point a lane) and closes it, while
  // that bound is at or below the query's best.  A skipped cell holds no
  // point whose distance is at most the best, so neither a smaller distance
  // nor a tie with a lower index is missed.  Same keys as the walk.
  if (const uint64_t farm = __ballot(far)) {
    float csc[3];
    int gac[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      csc[a] = U(__builtin_ldexpf(h[9 + a], 2));
      gac[a] = gs[a] > 0.f ? 8 : 1;
    }
    // distance from x to coarse cell c's slab along axis a, as axis_gap
    auto gap = [&](int a, int c, float x) {
      const float clo = (cut >> a) & 1u && c == 0
                            ? -__builtin_inff()
                            : (gac[a] > 1 ? glo[a] + (float)c * csc[a] : glo[a]) - eps[a];
      const float chi = (cut >> (3 + a)) & 1u && c == gac[a] - 1
                            ? __builtin_inff()
                            : (gac[a] > 1 ? glo[a] + (float)(c + 1) * csc[a] : ghi[a]) + eps[a];
      return fmaxf(fmaxf(clo - x, x - chi), 0.f);
    };
    // bit k: coarse cell lane + 64 k holds points
    uint32_t busy = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int c = lane + 64 * k, cx = c & 7, cy = (c >> 3) & 7, cz = c >> 6;
      const uint32_t code = cg_code(cx, cy, cz);
      if (cx < gac[0] && cy < gac[1] && cz < gac[2] &&
          cstart[(code + 1) << 6] > cstart[code << 6])
        busy |= 1u << k;
    }
    for (uint64_t fm = farm; fm; fm &= fm - 1) {
      const int l = __builtin_ctzll(fm);
      const float4 qf = wq[l];
      const float4 ql = make_float4(0.f, qf.x, qf.y, qf.z);
      unsigned long long key = wkey[l];
      uint32_t open = busy;  // bit k: not scanned yet for this query
      for (;;) {
        const float bd = __uint_as_float((uint32_t)(key >> 32));
        float m = __builtin_inff();
        int mk = -1;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int c = lane + 64 * k;
          const float b = fmaxf(sq3(gap(0, c & 7, qf.x), gap(1, (c >> 3) & 7, qf.y),
                                    gap(2, c >> 6, qf.z)) * Mg::lb - Mg::abs, 0.f);
          if ((open >> k) & 1u && (mk < 0 || b < m)) {  // an infinite bound is a bound too
            m = b;
            mk = k;
          }
        }
        // (bound, lane, cell) of the lane's nearest open cell; all ones when
        // it has none, above any open cell's key
        unsigned long long pk = mk < 0 ? ~0ull
                                       : (unsigned long long)__float_as_uint(m) << 32 |
                                             (uint32_t)(lane << 3 | mk);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          const unsigned long long x = __shfl_xor(pk, o);
          pk = x < pk ? x : pk;
        }
        // every round closes one open cell: at most 512 rounds.  No open cell
        // left, or the nearest above the best (an infinite best -- half
        // distances can overflow -- takes every cell): done
        if (pk == ~0ull || __uint_as_float((uint32_t)(pk >> 32)) > bd) break;
        const int wl = (int)(pk >> 3) & 63, wk = (int)pk & 7;
        if (lane == wl) open &= ~(1u << wk);
        const int c = __builtin_amdgcn_readfirstlane(wl + 64 * wk);
        const uint32_t code = cg_code(c & 7, (c >> 3) & 7, c >> 6);
        const int s0 = cstart[code << 6], s1 = cstart[(code + 1) << 6];
        examined += s1 - s0;
        unsigned long long kk = kInit;
        for (int j = s0 + lane; j < s1; j += 64) {
          const float4 p = rs[j];
          const unsigned long long k2 =
              ((unsigned long long)__float_as_uint(cg_dist<T>(p, ql)) << 32) | __float_as_uint(p.x);
          kk = k2 < kk ? k2 : kk;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          const unsigned long long x = __shfl_xor(kk, o);
          kk = x < kk ? x : kk;
        }
        key = kk < key ? kk : key;
      }
      if (lane == l) {
        dout[__float_as_int(qf.w)] = (T)__uint_as_float((uint32_t)(key >> 32));
        iout[__float_as_int(qf.w)] = (int)(uint32_t)key;
      }
    }
  }
  // points evaluated by this wave (a wave-uniform count)
  if (lane == 0) stats[(size_t)bid * (WG / 64) + w] = examined;
  // queries that need the reference's full rule: the wave scans one at a time
  uint64_t fb = __ballot(fallback);
  while (fb) {
    const int l = __builtin_ctzll(fb);
    fb &= fb - 1;
    const int o = __float_as_int(wq[l].w);
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
    hipLaunchKernelGGL((chamfer_grid_sort_kernel<T, 8>), dim3(4 * B), dim3(1024), 0, s,
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
