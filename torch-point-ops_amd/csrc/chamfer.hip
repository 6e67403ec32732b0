// chamfer.hip -- Chamfer distance forward/backward for gfx950.
//
// Forward (replaces chamfer_dist_kernel, chamfer.cu:36-167).
//   One launch covers both directions.  A workgroup owns 64*Q query points
//   (Q per lane, held in VGPRs) of one (direction, cloud) and its 4 waves split
//   the reference cloud into 4 contiguous chunks; chunk results merge in LDS in
//   index order with strict-less, so ties go to the lowest index -- the
//   reference's rule (chamfer.cu:69-72, 159-162).
//   float: chamfer_fwd_filter_kernel ranks references by the expanded form
//   |r|^2 - 2 q.r (3 FMAs per pair) and proves with a per-query error window
//   that the reference formula's first-index minimum lies in the best tile of
//   16, which it then re-scans exactly; queries the window cannot decide are
//   re-scanned exactly by the whole wave.
//   double / half: chamfer_fwd_kernel evaluates the reference formula per
//   pair (3 sub, mul, 2 fma, streamed through SGPRs), keeps only per-tile
//   minima and re-scans the winning tile for the first index.
//   Non-finite coordinates take the exact wave-wide scan, which follows the
//   reference's handling of NaN distances (chunk_scan).
// Backward (replaces chamfer_dist_grad_kernel, chamfer.cu:200-234).
//   grad_q[i] = 2 g_i (q_i - r_idx[i]) - sum over the other cloud's points j
//   matched to i of 2 g_j (r_j - q_i).  float/half: a workgroup per (batch,
//   cloud, slice of <= 4096 points) holds the slice's gradient in LDS,
//   accumulates the scattered terms that land in it with LDS atomics, adds
//   its points' direct terms and writes every element once: no global
//   atomics, no zero-fill.
//   (float16: terms are computed in half like the reference, accumulated in
//   float and rounded once.)  Otherwise pass 1 stores the direct terms (which
//   initialises both outputs) and pass 2 scatters the negated terms with
//   hardware atomics, like the reference.
#include <stdio.h>

#include <algorithm>
#include <mutex>

#include "chamfer_common.hpp"
#include "chamfer_dense.hpp"
#include "tpo_common.hpp"

#pragma clang fp contract(off)

namespace tpo {

// Block decode shared by the dense kernels: workgroup -> (direction,
// cloud, query block).
struct DenseBlock {
  int dir, b, qb, nq, nr;
};
__device__ __forceinline__ DenseBlock dense_block(int B, int N, int M, int nqb1, int nqb2) {
  int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int g1 = B * nqb1;
  DenseBlock d;
  d.dir = lb >= g1;
  if (d.dir) lb -= g1;
  const int nqb = d.dir ? nqb2 : nqb1;
  d.b = lb / nqb;
  d.qb = lb - d.b * nqb;
  d.nq = d.dir ? M : N;
  d.nr = d.dir ? N : M;
  return d;
}

template <typename T, int Q>
__global__ __launch_bounds__(256) void chamfer_fwd_kernel(
    const T* __restrict__ xyz1, const T* __restrict__ xyz2, int B, int N, int M, int nqb1,
    int nqb2, T* __restrict__ dist1, T* __restrict__ dist2, int32_t* __restrict__ idx1,
    int32_t* __restrict__ idx2) {
  __shared__ T s_d[CH_WAVES][64 * Q];
  __shared__ int s_i[CH_WAVES][64 * Q];
  const DenseBlock d = dense_block(B, N, M, nqb1, nqb2);
  chamfer_dense_block<T, Q>((d.dir ? xyz2 : xyz1) + (size_t)d.b * d.nq * 3,
                            (d.dir ? xyz1 : xyz2) + (size_t)d.b * d.nr * 3, d.nq, d.nr, d.qb,
                            (d.dir ? dist2 : dist1) + (size_t)d.b * d.nq,
                            (d.dir ? idx2 : idx1) + (size_t)d.b * d.nq, s_d, s_i);
}

template <int Q, int TT>
__global__ __launch_bounds__(256) void chamfer_fwd_filter_kernel(
    const float* __restrict__ xyz1, const float* __restrict__ xyz2, int B, int N, int M,
    int nqb1, int nqb2, float* __restrict__ dist1, float* __restrict__ dist2,
    int32_t* __restrict__ idx1, int32_t* __restrict__ idx2) {
  __shared__ float4 s_ref[CH_WAVES][64];
  __shared__ float s_d[CH_WAVES][64 * Q];
  __shared__ int s_i[CH_WAVES][64 * Q];
  const DenseBlock d = dense_block(B, N, M, nqb1, nqb2);
  chamfer_filter_block<Q, TT>((d.dir ? xyz2 : xyz1) + (size_t)d.b * d.nq * 3,
                              (d.dir ? xyz1 : xyz2) + (size_t)d.b * d.nr * 3, d.nq, d.nr, d.qb,
                              (d.dir ? dist2 : dist1) + (size_t)d.b * d.nq,
                              (d.dir ? idx2 : idx1) + (size_t)d.b * d.nq, s_ref, s_d, s_i);
}

// ---------------------------------------------------------------- backward
// Upstream gradient of one cloud's distances: one value per point, or (the
// loss entry points) the loss gradient spread over every point the way
// torch's autograd does it for the module's reduction -- MeanBackward
// multiplies by 1 / numel in the accumulation type, SumBackward copies.
template <typename T>
struct PointGrad {
  const T* __restrict__ p;  // per point, or the single loss gradient
  int64_t count;            // 0: per point; > 0: mean over count points; < 0: sum
  __device__ __forceinline__ bool uniform() const { return count != 0; }
  __device__ __forceinline__ T spread() const {  // the per-point value (uniform only)
    using A = typename std::conditional<sizeof(T) == 8, double, float>::type;
    return count > 0 ? (T)((A)p[0] * ((A)1 / (A)count)) : p[0];
  }
};

// Pass 1: grad_q[i] = g (q_i - r_idx[i]) with g = 2 grad_dist[i] (in dtype);
// every element of both outputs is written here.
template <typename T>
__global__ __launch_bounds__(256) void chamfer_bwd_direct_kernel(
    const T* __restrict__ xyz1, const T* __restrict__ xyz2, const int32_t* __restrict__ idx1,
    const int32_t* __restrict__ idx2, PointGrad<T> gd1, PointGrad<T> gd2, int64_t B, int64_t N,
    int64_t M, T* __restrict__ g1, T* __restrict__ g2) {
  const int64_t n1 = B * N, total = n1 + B * M;
  const T u1 = gd1.uniform() ? gd1.spread() : (T)0, u2 = gd2.uniform() ? gd2.spread() : (T)0;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const bool dir = t >= n1;
    const int64_t u = dir ? t - n1 : t;
    const int64_t nq = dir ? M : N, nr = dir ? N : M;
    const int64_t b = u / nq;
    const T* q = dir ? xyz2 : xyz1;
    const T* r = dir ? xyz1 : xyz2;
    const int64_t j2 = (dir ? idx2 : idx1)[u];
    T* go = dir ? g2 : g1;
    T cx = (T)0, cy = (T)0, cz = (T)0;
    if (j2 >= 0 && j2 < nr) {
      const PointGrad<T> gd = dir ? gd2 : gd1;
      const T g = (T)((gd.uniform() ? (dir ? u2 : u1) : gd.p[u]) * (T)2);
      const int64_t ro = (b * nr + j2) * 3;
      cx = (T)(g * (T)(q[3 * u] - r[ro]));
      cy = (T)(g * (T)(q[3 * u + 1] - r[ro + 1]));
      cz = (T)(g * (T)(q[3 * u + 2] - r[ro + 2]));
    }
    go[3 * u] = cx;
    go[3 * u + 1] = cy;
    go[3 * u + 2] = cz;
  }
}

// Pass 2: grad_r[idx[i]] += -(g (q_i - r_idx[i])), atomically.
template <typename T>
__global__ __launch_bounds__(256) void chamfer_bwd_scatter_kernel(
    const T* __restrict__ xyz1, const T* __restrict__ xyz2, const int32_t* __restrict__ idx1,
    const int32_t* __restrict__ idx2, PointGrad<T> gd1, PointGrad<T> gd2, int64_t B, int64_t N,
    int64_t M, T* __restrict__ g1, T* __restrict__ g2) {
  const int64_t n1 = B * N, total = n1 + B * M;
  const T u1 = gd1.uniform() ? gd1.spread() : (T)0, u2 = gd2.uniform() ? gd2.spread() : (T)0;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const bool dir = t >= n1;
    const int64_t u = dir ? t - n1 : t;
    const int64_t nq = dir ? M : N, nr = dir ? N : M;
    const int64_t b = u / nq;
    const T* q = dir ? xyz2 : xyz1;
    const T* r = dir ? xyz1 : xyz2;
    const int64_t j2 = (dir ? idx2 : idx1)[u];
    if (j2 < 0 || j2 >= nr) continue;
    T* gr = dir ? g1 : g2;
    const PointGrad<T> gd = dir ? gd2 : gd1;
    const T g = (T)((gd.uniform() ? (dir ? u2 : u1) : gd.p[u]) * (T)2);
    const int64_t ro = (b * nr + j2) * 3;
    atomic_add(gr + ro, (T)(-(T)(g * (T)(q[3 * u] - r[ro]))));
    atomic_add(gr + ro + 1, (T)(-(T)(g * (T)(q[3 * u + 1] - r[ro + 1]))));
    atomic_add(gr + ro + 2, (T)(-(T)(g * (T)(q[3 * u + 2] - r[ro + 2]))));
  }
}

// One workgroup per (batch, cloud, slice of that cloud's points): the slice's
// gradient rows and coordinates live in LDS; the workgroup scans the other
// cloud's nearest indices and accumulates, with LDS atomics, the terms that
// land in its slice; then it adds its points' direct terms and writes each
// element once.  The scan's loads do not depend on the indices (VEC: four
// consecutive points per lane, one 16-byte index load and three 16-byte
// coordinate loads), so they are all in flight together; only the LDS
// atomics are conditional.
constexpr int CH_BWD_SLICE_MAX = 4096;  // points per slice (96 KiB of LDS)
constexpr int CH_BWD_MAX_SLICES = 16;   // beyond this the 2-pass path is cheaper
constexpr int CH_BWD_THREADS = 512;     // threads per workgroup
constexpr int CH_BWD_PF = 2;            // own points per thread prefetched for the direct term

template <typename T, bool VEC>
__global__ __launch_bounds__(CH_BWD_THREADS) void chamfer_bwd_fused_kernel(
    const T* __restrict__ xyz1, const T* __restrict__ xyz2, const int32_t* __restrict__ idx1,
    const int32_t* __restrict__ idx2, PointGrad<T> gd1, PointGrad<T> gd2, int N, int M, int S,
    T* __restrict__ g1, T* __restrict__ g2) {
  extern __shared__ float sm[];
  int b, c, sl;  // batch, cloud (0: gradient of cloud 1, 1: of cloud 2), slice
  {
    int j;
    if (batch_home_block(blockIdx.x, gridDim.x / (2 * S), 2 * S, b, j)) {
      c = j / S;
      sl = j - c * S;
    } else {
      const int lb = xcd_logical_block(blockIdx.x, gridDim.x);
      sl = lb % S;
      c = (lb / S) & 1;
      b = lb / (2 * S);
    }
  }
  const int n_own = c ? M : N, n_oth = c ? N : M;
  const int span = (n_own + S - 1) / S;
  const int lo = min(n_own, sl * span), hi = min(n_own, lo + span);
  float* __restrict__ acc = sm;                 // 3 * span
  float* __restrict__ s_own = sm + 3 * span;    // the slice's coordinates
  const T* __restrict__ own = (c ? xyz2 : xyz1) + (size_t)b * n_own * 3;
  const T* __restrict__ oth = (c ? xyz1 : xyz2) + (size_t)b * n_oth * 3;
  const int32_t* __restrict__ idx_own = (c ? idx2 : idx1) + (size_t)b * n_own;
  const int32_t* __restrict__ idx_oth = (c ? idx1 : idx2) + (size_t)b * n_oth;
  const PointGrad<T> pg_own = c ? gd2 : gd1, pg_oth = c ? gd1 : gd2;
  const bool uni_own = pg_own.uniform(), uni_oth = pg_oth.uniform();
  const T u_own = uni_own ? pg_own.spread() : (T)0, u_oth = uni_oth ? pg_oth.spread() : (T)0;
  const T* __restrict__ gd_own = pg_own.p + (uni_own ? 0 : (size_t)b * n_own);
  const T* __restrict__ gd_oth = pg_oth.p + (uni_oth ? 0 : (size_t)b * n_oth);
  T* __restrict__ out = (c ? g2 : g1) + (size_t)b * n_own * 3;

  // Every phase issues all of its loads before it waits on any: the
  // direct-term inputs of the first CH_BWD_PF points per thread (their nearest
  // indices, then the other cloud's coordinates at them, which land during
  // the staging and the scan), and the slice's coordinates for LDS, 8 values
  // a thread per round.
  int pj[CH_BWD_PF];
  T pg[CH_BWD_PF], po[CH_BWD_PF][3];
#pragma unroll
  for (int u = 0; u < CH_BWD_PF; ++u) {
    const int i = lo + (int)threadIdx.x + CH_BWD_THREADS * u;
    pj[u] = i < hi ? idx_own[i] : -1;
    pg[u] = i < hi ? (T)((uni_own ? u_own : gd_own[i]) * (T)2) : (T)0;
  }
  const int nv = 3 * (hi - lo);
  const T* __restrict__ own_s = own + 3 * lo;
  for (int t0 = 0; t0 < nv; t0 += CH_BWD_THREADS * 8) {
    T v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int t = t0 + (int)threadIdx.x + CH_BWD_THREADS * u;
      v[u] = t < nv ? own_s[t] : (T)0;
    }
    if (t0 == 0) {
#pragma unroll
      for (int u = 0; u < CH_BWD_PF; ++u) {
        const bool ok = pj[u] >= 0 && pj[u] < n_oth;
        pj[u] = ok ? pj[u] : -1;
#pragma unroll
        for (int k = 0; k < 3; ++k) po[u][k] = ok ? oth[3 * pj[u] + k] : (T)0;
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int t = t0 + (int)threadIdx.x + CH_BWD_THREADS * u;
      if (t < nv) {
        acc[t] = 0.f;
        s_own[t] = (float)v[u];
      }
    }
  }
  if (nv == 0) {
#pragma unroll
    for (int u = 0; u < CH_BWD_PF; ++u) pj[u] = -1;
  }
  __syncthreads();
  // other cloud's point j whose nearest point i is in [lo, hi)
  // (chamfer.cu:229-231 of the other direction): acc[i] += -(g_j (r_j - q_i))
  auto scatter = [&](int j, int i, T rx, T ry, T rz, T gj) {
    if (i < lo || i >= hi) return;
    const T g = (T)(gj * (T)2);
    const int a = 3 * (i - lo);
    atomicAdd(&acc[a], -(float)(T)(g * (T)(rx - (T)s_own[a])));
    atomicAdd(&acc[a + 1], -(float)(T)(g * (T)(ry - (T)s_own[a + 1])));
    atomicAdd(&acc[a + 2], -(float)(T)(g * (T)(rz - (T)s_own[a + 2])));
  };
  if constexpr (VEC) {  // float, n_oth % 4 == 0, 16-byte aligned rows
    const int4* __restrict__ iv = reinterpret_cast<const int4*>(idx_oth);
    const float4* __restrict__ rv = reinterpret_cast<const float4*>(oth);
    const float4* __restrict__ gv = reinterpret_cast<const float4*>(gd_oth);
    // four groups of four points per thread: all their loads before the
    // first scatter
    constexpr int U = 4;
    const int nq4 = n_oth / 4;
    for (int q0 = threadIdx.x; q0 < nq4; q0 += CH_BWD_THREADS * U) {
      int4 ii[U];
      float4 r[U][3], gg[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = min(q0 + CH_BWD_THREADS * u, nq4 - 1);  // a repeat is not scattered
        ii[u] = iv[q];
        r[u][0] = rv[3 * q];
        r[u][1] = rv[3 * q + 1];
        r[u][2] = rv[3 * q + 2];
        gg[u] = uni_oth ? make_float4(u_oth, u_oth, u_oth, u_oth) : gv[q];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = q0 + CH_BWD_THREADS * u;
        if (q >= nq4) break;
        scatter(4 * q, ii[u].x, r[u][0].x, r[u][0].y, r[u][0].z, gg[u].x);
        scatter(4 * q + 1, ii[u].y, r[u][0].w, r[u][1].x, r[u][1].y, gg[u].y);
        scatter(4 * q + 2, ii[u].z, r[u][1].z, r[u][1].w, r[u][2].x, gg[u].z);
        scatter(4 * q + 3, ii[u].w, r[u][2].y, r[u][2].z, r[u][2].w, gg[u].w);
      }
    }
  } else {
#pragma unroll 4
    for (int j = threadIdx.x; j < n_oth; j += CH_BWD_THREADS)
      scatter(j, idx_oth[j], oth[3 * j], oth[3 * j + 1], oth[3 * j + 2],
              uni_oth ? u_oth : gd_oth[j]);
  }
  __syncthreads();
  // direct term of the slice's points (chamfer.cu:226-228)
#pragma unroll
  for (int u = 0; u < CH_BWD_PF; ++u) {
    const int i = lo + (int)threadIdx.x + CH_BWD_THREADS * u;
    if (i >= hi) break;
    const int a = 3 * (i - lo);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const T d = pj[u] >= 0 ? (T)(pg[u] * (T)((T)s_own[a + k] - po[u][k])) : (T)0;
      out[3 * i + k] = (T)(acc[a + k] + (float)d);
    }
  }
  for (int i = lo + (int)threadIdx.x + CH_BWD_THREADS * CH_BWD_PF; i < hi;
       i += CH_BWD_THREADS) {
    const int j2 = idx_own[i];
    const bool ok = j2 >= 0 && j2 < n_oth;
    const int jj = ok ? j2 : 0;
    const T g = (T)((uni_own ? u_own : gd_own[i]) * (T)2);
    const int a = 3 * (i - lo);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const T d = ok ? (T)(g * (T)((T)s_own[a + k] - oth[3 * jj + k])) : (T)0;
      out[3 * i + k] = (T)(acc[a + k] + (float)d);
    }
  }
}

template <typename T, int Q>
static void launch_fwd(const void* x1, const void* x2, int B, int N, int M, void* d1, void* d2,
                       int32_t* i1, int32_t* i2, hipStream_t s) {
  const int nqb1 = (N + 64 * Q - 1) / (64 * Q), nqb2 = (M + 64 * Q - 1) / (64 * Q);
  const int grid = B * (nqb1 + nqb2);
  if (grid == 0) return;
  hipLaunchKernelGGL((chamfer_fwd_kernel<T, Q>), dim3(grid), dim3(256), 0, s, (const T*)x1,
                     (const T*)x2, B, N, M, nqb1, nqb2, (T*)d1, (T*)d2, i1, i2);
}

template <int Q, int TT>
static void launch_fwd_filter(const void* x1, const void* x2, int B, int N, int M, void* d1,
                              void* d2, int32_t* i1, int32_t* i2, hipStream_t s) {
  const int nqb1 = (N + 64 * Q - 1) / (64 * Q), nqb2 = (M + 64 * Q - 1) / (64 * Q);
  const int grid = B * (nqb1 + nqb2);
  if (grid == 0) return;
  hipLaunchKernelGGL((chamfer_fwd_filter_kernel<Q, TT>), dim3(grid), dim3(256), 0, s,
                     (const float*)x1, (const float*)x2, B, N, M, nqb1, nqb2, (float*)d1,
                     (float*)d2, i1, i2);
}

template <typename T>
static void fwd_dispatch(const void* x1, const void* x2, int B, int N, int M, void* d1, void* d2,
                         int32_t* i1, int32_t* i2, hipStream_t s) {
  // Largest per-lane query count that still gives >= 2 workgroups per CU.
  const int64_t q = (int64_t)B * ((int64_t)N + M);
  if constexpr (sizeof(T) == 4) {
    if (q >= (int64_t)512 * 64 * 8) launch_fwd_filter<8, CH_FTILE>(x1, x2, B, N, M, d1, d2, i1, i2, s);
    else if (q >= (int64_t)512 * 64 * 4) launch_fwd_filter<4, CH_FTILE>(x1, x2, B, N, M, d1, d2, i1, i2, s);
    else if (q >= (int64_t)512 * 64 * 2) launch_fwd_filter<2, CH_FTILE>(x1, x2, B, N, M, d1, d2, i1, i2, s);
    else launch_fwd_filter<1, CH_FTILE>(x1, x2, B, N, M, d1, d2, i1, i2, s);
  } else {
    if (q >= (int64_t)512 * 64 * 8) launch_fwd<T, 8>(x1, x2, B, N, M, d1, d2, i1, i2, s);
    else if (q >= (int64_t)512 * 64 * 4) launch_fwd<T, 4>(x1, x2, B, N, M, d1, d2, i1, i2, s);
    else if (q >= (int64_t)512 * 64 * 2) launch_fwd<T, 2>(x1, x2, B, N, M, d1, d2, i1, i2, s);
    else launch_fwd<T, 1>(x1, x2, B, N, M, d1, d2, i1, i2, s);
  }
}


template <typename T>
static void bwd_dispatch(const void* x1, const void* x2, const int32_t* i1, const int32_t* i2,
                         const void* gd1, const void* gd2, int64_t B, int64_t N, int64_t M,
                         void* g1, void* g2, hipStream_t s, int64_t count1 = 0,
                         int64_t count2 = 0) {
  const int64_t total = B * (N + M);
  if (total == 0) return;
  const PointGrad<T> pg1{(const T*)gd1, count1}, pg2{(const T*)gd2, count2};
  if (sizeof(T) <= 4) {
    // slices: enough for one cloud's slice to fit LDS and for ~512 workgroups
    const int64_t nmax = std::max(N, M);
    int64_t S = (nmax + CH_BWD_SLICE_MAX - 1) / CH_BWD_SLICE_MAX;
    const int64_t want = (512 + 2 * B - 1) / (2 * B);
    S = std::max(S, std::min({want, std::max<int64_t>(1, nmax / 512), (int64_t)CH_BWD_MAX_SLICES}));
    if (S <= CH_BWD_MAX_SLICES && 2 * B * S < (1 << 30)) {
      const int64_t span = (nmax + S - 1) / S;
      const size_t lds = (size_t)(6 * span * sizeof(float));
      auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
      const bool vec = sizeof(T) == 4 && N % 4 == 0 && M % 4 == 0 && al16(x1) && al16(x2) &&
                       al16(i1) && al16(i2) && (count1 != 0 || al16(gd1)) &&
                       (count2 != 0 || al16(gd2));
      if constexpr (sizeof(T) == 4) {
        if (vec) {
          hipLaunchKernelGGL((chamfer_bwd_fused_kernel<T, true>), dim3((unsigned)(2 * B * S)),
                             dim3(CH_BWD_THREADS), lds, s, (const T*)x1, (const T*)x2, i1, i2,
                             pg1, pg2,
                             (int)N, (int)M, (int)S, (T*)g1, (T*)g2);
          return;
        }
      }
      hipLaunchKernelGGL((chamfer_bwd_fused_kernel<T, false>), dim3((unsigned)(2 * B * S)),
                         dim3(CH_BWD_THREADS), lds, s, (const T*)x1, (const T*)x2, i1, i2, pg1,
                         pg2, (int)N,
                         (int)M, (int)S, (T*)g1, (T*)g2);
      return;
    }
  }
  const int64_t blocks = std::min<int64_t>((total + 255) / 256, 65536);
  hipLaunchKernelGGL(chamfer_bwd_direct_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, s,
                     (const T*)x1, (const T*)x2, i1, i2, pg1, pg2, B, N, M, (T*)g1, (T*)g2);
  hipLaunchKernelGGL(chamfer_bwd_scatter_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, s,
                     (const T*)x1, (const T*)x2, i1, i2, pg1, pg2, B, N, M, (T*)g1, (T*)g2);
}

// ------------------------------------------------------------------- loss
// The module's reduction (tpo_chamfer_loss_fwd): the forward stores both
// distance arrays in the workspace and chamfer_loss_part_kernel sums fixed
// chunks of them in original point order; the chunk sums are then added in
// a fixed order, by the last part workgroup to finish (LAST: the grid path,
// whose sort kernel zeroes the workgroup counter) or by
// chamfer_loss_final_kernel.  The loss therefore does not depend on how the
// forward scheduled its queries.  (A reduction inside the grid search, one
// sum per wave, would follow the search's query order, which the sort's
// arrival-order ranks make nondeterministic; and a device-scope release per
// search workgroup is an L2 writeback that evicts the reference points the
// other workgroups are reading.)
constexpr int CH_LOSS_PARTS = 256;       // chunks per array, at most
constexpr int64_t CH_LOSS_CHUNK = 4096;  // elements per chunk, at least

static int64_t loss_parts(int64_t n) {
  return std::min<int64_t>((n + CH_LOSS_CHUNK - 1) / CH_LOSS_CHUNK, CH_LOSS_PARTS);
}

// Loss from the chunk sums, by one wave: parts [0, p1) sum dist1,
// [p1, p1 + p2) dist2.  Lane 63 writes, as torch.mean / torch.sum of each
// array followed by their sum (chamfer.py:20-23; torch's mean scales the
// accumulated sum by 1 / numel in the accumulation type, and an empty
// array's mean is NaN):
//   mean: (T)(S1 * (1 / count1)) + (T)(S2 * (1 / count2))
//   sum:  (T)S1 + (T)S2
template <typename T>
__device__ void chamfer_loss_finish(const double* part, int p1, int p2, int mean, int64_t count1,
                                    int64_t count2, T* loss) {
  using A = typename std::conditional<sizeof(T) == 8, double, float>::type;
  const int lane = threadIdx.x & 63;
  A a1 = (A)0, a2 = (A)0;
  for (int k = lane; k < p1; k += 64) a1 += (A)part[k];
  for (int k = lane; k < p2; k += 64) a2 += (A)part[p1 + k];
  a1 = wave_add63(a1);
  a2 = wave_add63(a2);
  if (lane == 63) {
    if (mean) {
      a1 *= (A)1 / (A)count1;
      a2 *= (A)1 / (A)count2;
    }
    loss[0] = (T)((A)(T)a1 + (A)(T)a2);
  }
}

template <typename T, bool LAST>
__global__ __launch_bounds__(256) void chamfer_loss_part_kernel(
    const T* __restrict__ d1, const T* __restrict__ d2, int64_t n1, int64_t n2, int p1, int p2,
    double* __restrict__ part, uint32_t* __restrict__ done, int mean, T* __restrict__ loss,
    int home_b, int home_c1, int home_c2) {
  using A = typename std::conditional<sizeof(T) == 8, double, float>::type;
  __shared__ A s_red[4];
  __shared__ int s_last;
  // chunk k of the arrays; with home_b > 0 (chunks aligned to the home_b
  // batches, home_c1 / home_c2 of them per batch and array) batch b's chunks
  // run on XCD b % 8, where the grid search wrote its distances
  int k = blockIdx.x;
  {
    int b, j;
    if (home_b > 0 && batch_home_block(blockIdx.x, home_b, home_c1 + home_c2, b, j))
      k = j < home_c1 ? b * home_c1 + j : p1 + b * home_c2 + (j - home_c1);
  }
  const bool second = k >= p1;
  const T* d = second ? d2 : d1;
  const int64_t n = second ? n2 : n1;
  const int np = second ? p2 : p1, kk = second ? k - p1 : k;
  const int64_t chunk = (n + np - 1) / np;
  const int64_t lo = kk * chunk < n ? kk * chunk : n, hi = lo + chunk < n ? lo + chunk : n;
  A a = (A)0;
#pragma unroll 8
  for (int64_t i = lo + threadIdx.x; i < hi; i += 256) a += (A)d[i];
  a = wave_add63(a);
  if ((threadIdx.x & 63) == 63) s_red[threadIdx.x >> 6] = a;
  __syncthreads();
  if (threadIdx.x == 0) part[k] = (double)(((s_red[0] + s_red[1]) + s_red[2]) + s_red[3]);
  if constexpr (LAST) {
    // publish the chunk sum (device-scope release), count the workgroup;
    // the last one acquires every chunk sum and finishes the loss
    if (threadIdx.x == 0) {
      __threadfence();
      s_last = atomicAdd(done, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (s_last && threadIdx.x < 64) {
      __threadfence();
      chamfer_loss_finish<T>(part, p1, p2, mean, n1, n2, loss);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(64) void chamfer_loss_final_kernel(const double* __restrict__ part,
                                                                int p1, int p2, int mean,
                                                                int64_t count1, int64_t count2,
                                                                T* __restrict__ loss) {
  chamfer_loss_finish<T>(part, p1, p2, mean, count1, count2, loss);
}

// Workspace of tpo_chamfer_loss_fwd:
// [forward workspace][dist1][dist2][chunk sums][workgroup counter].
struct LossLayout {
  int64_t fwd, d1, d2, part, done, total;
};

static LossLayout loss_layout(int64_t fwd_bytes, int64_t esize, int64_t B, int64_t N, int64_t M) {
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  LossLayout L;
  L.fwd = 0;
  L.d1 = up(fwd_bytes);
  L.d2 = L.d1 + up(B * N * esize);
  L.part = L.d2 + up(B * M * esize);
  L.done = L.part + up(2 * CH_LOSS_PARTS * 8);
  L.total = L.done + 256;
  return L;
}

// counter_zeroed: the forward's sort kernel has set the counter to 0, so the
// part kernel can finish the loss itself (one launch instead of two).
template <typename T>
static void loss_reduce(const LossLayout& L, char* ws, int64_t B, int64_t N, int64_t M, int mean,
                        void* loss, bool counter_zeroed, hipStream_t s) {
  const T* d1 = (const T*)(ws + L.d1);
  const T* d2 = (const T*)(ws + L.d2);
  double* part = (double*)(ws + L.part);
  uint32_t* done = (uint32_t*)(ws + L.done);
  const int p1 = (int)loss_parts(B * N), p2 = (int)loss_parts(B * M);
  // chunks aligned to batches (the grid search's batch-per-XCD order)
  const bool home = B > 0 && B <= (1 << 20) && N % CH_LOSS_CHUNK == 0 && M % CH_LOSS_CHUNK == 0 &&
                    p1 == B * N / CH_LOSS_CHUNK && p2 == B * M / CH_LOSS_CHUNK;
  const int hb = home ? (int)B : 0;
  const int hc1 = home ? (int)(N / CH_LOSS_CHUNK) : 0, hc2 = home ? (int)(M / CH_LOSS_CHUNK) : 0;
  if (counter_zeroed && p1 + p2 > 0) {
    hipLaunchKernelGGL((chamfer_loss_part_kernel<T, true>), dim3(p1 + p2), dim3(256), 0, s, d1,
                       d2, B * N, B * M, p1, p2, part, done, mean, (T*)loss, hb, hc1, hc2);
    return;
  }
  if (p1 + p2 > 0)
    hipLaunchKernelGGL((chamfer_loss_part_kernel<T, false>), dim3(p1 + p2), dim3(256), 0, s, d1,
                       d2, B * N, B * M, p1, p2, part, done, mean, (T*)loss, hb, hc1, hc2);
  hipLaunchKernelGGL(chamfer_loss_final_kernel<T>, dim3(1), dim3(64), 0, s, part, p1, p2, mean,
                     B * N, B * M, (T*)loss);
}

}  // namespace tpo

using namespace tpo;

static bool prune_applies(int dtype, int64_t B, int64_t N, int64_t M) {
  return (dtype == TPO_F32 || dtype == TPO_F16) && B > 0 && N >= CH_PRUNE_MIN &&
         M >= CH_PRUNE_MIN;
}

extern "C" int64_t tpo_chamfer_workspace_size(int dtype, int64_t B, int64_t N, int64_t M) {
  if (B < 0 || N < 0 || M < 0) return -1;
  return prune_applies(dtype, B, N, M) ? chamfer_prune_workspace(B, N, M) : 0;
}

extern "C" int tpo_chamfer_fwd(int dtype, const void* xyz1, const void* xyz2, int64_t B,
                               int64_t N, int64_t M, void* dist1, void* dist2, int32_t* idx1,
                               int32_t* idx2, void* workspace, int64_t workspace_bytes,
                               void* stream) {
  if (B < 0 || N < 0 || M < 0 || N >= (1 << 28) || M >= (1 << 28) ||
      B * (N + M) >= ((int64_t)1 << 31))
    return set_error(TPO_ERR_ARG, "tpo_chamfer_fwd: bad sizes B=%lld N=%lld M=%lld",
                     (long long)B, (long long)N, (long long)M);
  if (B == 0 || (N == 0 && M == 0)) return TPO_OK;
  if ((N > 0 && (!xyz1 || !dist1 || !idx1)) || (M > 0 && (!xyz2 || !dist2 || !idx2)))
    return set_error(TPO_ERR_ARG, "tpo_chamfer_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (workspace && prune_applies(dtype, B, N, M)) {
    const int64_t need = chamfer_prune_workspace(B, N, M);
    if (workspace_bytes < need)
      return set_error(TPO_ERR_WORKSPACE, "tpo_chamfer_fwd: workspace of %lld bytes < %lld",
                       (long long)workspace_bytes, (long long)need);
    launch_chamfer_fwd_prune(dtype, xyz1, xyz2, (int)B, (int)N, (int)M, dist1, dist2, idx1,
                             idx2, workspace, s);
    return check_launch("tpo_chamfer_fwd");
  }
  switch (dtype) {
    case TPO_F32: fwd_dispatch<float>(xyz1, xyz2, (int)B, (int)N, (int)M, dist1, dist2, idx1, idx2, s); break;
    case TPO_F64: fwd_dispatch<double>(xyz1, xyz2, (int)B, (int)N, (int)M, dist1, dist2, idx1, idx2, s); break;
    case TPO_F16: fwd_dispatch<half_t>(xyz1, xyz2, (int)B, (int)N, (int)M, dist1, dist2, idx1, idx2, s); break;
    default: return set_error(TPO_ERR_DTYPE, "tpo_chamfer_fwd: unsupported dtype %d", dtype);
  }
  return check_launch("tpo_chamfer_fwd");
}

// ---------------------------------------------------------------------------
// Allocation-free forward.  The grid-search workspace lives in a file-scope
// device array: every GPU the library runs on holds its own copy (allocated
// when the code object is loaded on that device) until the process ends.
// Host code never passes `scratch` itself (in host code the name is a
// stand-in, not a device address): each device's address is looked up once
// with hipGetSymbolAddress and kept per device.  Every call on a device
// shares its array, so calls that overlap on one GPU (different streams, or
// threads) race; calls in one stream are ordered.  Nothing in it needs to
// start at zero: the sort kernel writes every region the search reads.
static constexpr int64_t kNoAllocScratchBytes = (int64_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];
}  // namespace

static int noalloc_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(TPO_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(TPO_ERR_ARG, "tpo_chamfer_fwd_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(TPO_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TPO_OK;
}

extern "C" int64_t tpo_chamfer_noalloc_max_workspace(void) { return kNoAllocScratchBytes; }

extern "C" int tpo_chamfer_fwd_noalloc(int dtype, const void* xyz1, const void* xyz2, int64_t B,
                                       int64_t N, int64_t M, void* dist1, void* dist2,
                                       int32_t* idx1, int32_t* idx2, void* stream) {
  const int64_t need = tpo_chamfer_workspace_size(dtype, B, N, M);
  if (need < 0)
    return set_error(TPO_ERR_ARG, "tpo_chamfer_fwd_noalloc: bad sizes B=%lld N=%lld M=%lld",
                     (long long)B, (long long)N, (long long)M);
  if (need > kNoAllocScratchBytes)
    return set_error(TPO_ERR_WORKSPACE,
                     "tpo_chamfer_fwd_noalloc: B=%lld N=%lld M=%lld needs %lld bytes of grid "
                     "workspace, more than the %lld-byte static scratch (use tpo_chamfer_fwd "
                     "with a caller-provided workspace)",
                     (long long)B, (long long)N, (long long)M, (long long)need,
                     (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = noalloc_scratch(&ws);
    if (rc != TPO_OK) return rc;
  }
  return tpo_chamfer_fwd(dtype, xyz1, xyz2, B, N, M, dist1, dist2, idx1, idx2, ws, need, stream);
}

extern "C" int tpo_chamfer_pairs_evaluated(int dtype, const void* workspace, int64_t B,
                                           int64_t N, int64_t M, int64_t* pairs, void* stream) {
  if (!workspace || !pairs || !prune_applies(dtype, B, N, M))
    return set_error(TPO_ERR_ARG,
                     "tpo_chamfer_pairs_evaluated: no pruned forward for these arguments");
  launch_chamfer_prune_stats(workspace, B, N, M, pairs, (hipStream_t)stream);
  return check_launch("tpo_chamfer_pairs_evaluated");
}

extern "C" int tpo_chamfer_bwd(int dtype, const void* xyz1, const void* xyz2,
                               const int32_t* idx1, const int32_t* idx2, const void* gd1,
                               const void* gd2, int64_t B, int64_t N, int64_t M, void* gxyz1,
                               void* gxyz2, void* stream) {
  if (B < 0 || N < 0 || M < 0 || B * (N + M) >= ((int64_t)1 << 40))
    return set_error(TPO_ERR_ARG, "tpo_chamfer_bwd: bad sizes");
  if (B == 0 || (N == 0 && M == 0)) return TPO_OK;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case TPO_F32: bwd_dispatch<float>(xyz1, xyz2, idx1, idx2, gd1, gd2, B, N, M, gxyz1, gxyz2, s); break;
    case TPO_F64: bwd_dispatch<double>(xyz1, xyz2, idx1, idx2, gd1, gd2, B, N, M, gxyz1, gxyz2, s); break;
    case TPO_F16: bwd_dispatch<half_t>(xyz1, xyz2, idx1, idx2, gd1, gd2, B, N, M, gxyz1, gxyz2, s); break;
    default: return set_error(TPO_ERR_DTYPE, "tpo_chamfer_bwd: unsupported dtype %d", dtype);
  }
  return check_launch("tpo_chamfer_bwd");
}

static int64_t esize_of(int dtype) {
  return dtype == TPO_F32 ? 4 : dtype == TPO_F64 ? 8 : dtype == TPO_F16 ? 2 : -1;
}

static LossLayout loss_layout_for(int dtype, int64_t B, int64_t N, int64_t M) {
  const int64_t fwd = prune_applies(dtype, B, N, M) ? chamfer_prune_workspace(B, N, M) : 0;
  return loss_layout(fwd, esize_of(dtype), B, N, M);
}

extern "C" int64_t tpo_chamfer_loss_workspace_size(int dtype, int64_t B, int64_t N, int64_t M) {
  if (B < 0 || N < 0 || M < 0 || esize_of(dtype) < 0) return -1;
  return loss_layout_for(dtype, B, N, M).total;
}

extern "C" int tpo_chamfer_loss_fwd(int dtype, const void* xyz1, const void* xyz2, int64_t B,
                                    int64_t N, int64_t M, int mean, void* loss, int32_t* idx1,
                                    int32_t* idx2, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
  if (B < 0 || N < 0 || M < 0 || N >= (1 << 28) || M >= (1 << 28) ||
      B * (N + M) >= ((int64_t)1 << 31))
    return set_error(TPO_ERR_ARG, "tpo_chamfer_loss_fwd: bad sizes B=%lld N=%lld M=%lld",
                     (long long)B, (long long)N, (long long)M);
  if (!loss || (B > 0 && ((N > 0 && (!xyz1 || !idx1)) || (M > 0 && (!xyz2 || !idx2)))))
    return set_error(TPO_ERR_ARG, "tpo_chamfer_loss_fwd: null pointer");
  if (esize_of(dtype) < 0)
    return set_error(TPO_ERR_DTYPE, "tpo_chamfer_loss_fwd: unsupported dtype %d", dtype);
  const LossLayout L = loss_layout_for(dtype, B, N, M);
  if (!workspace || workspace_bytes < L.total)
    return set_error(TPO_ERR_WORKSPACE, "tpo_chamfer_loss_fwd: workspace of %lld bytes < %lld",
                     (long long)(workspace ? workspace_bytes : 0), (long long)L.total);
  hipStream_t s = (hipStream_t)stream;
  char* w = (char*)workspace;
  void* d1 = w + L.d1;
  void* d2 = w + L.d2;
  const bool grid = B > 0 && N + M > 0 && prune_applies(dtype, B, N, M);
  if (B > 0 && N + M > 0) {
    if (grid)
      launch_chamfer_fwd_prune(dtype, xyz1, xyz2, (int)B, (int)N, (int)M, d1, d2, idx1, idx2,
                               w + L.fwd, s, (uint32_t*)(w + L.done));
    else if (dtype == TPO_F32)
      fwd_dispatch<float>(xyz1, xyz2, (int)B, (int)N, (int)M, d1, d2, idx1, idx2, s);
    else if (dtype == TPO_F64)
      fwd_dispatch<double>(xyz1, xyz2, (int)B, (int)N, (int)M, d1, d2, idx1, idx2, s);
    else
      fwd_dispatch<half_t>(xyz1, xyz2, (int)B, (int)N, (int)M, d1, d2, idx1, idx2, s);
  }
  switch (dtype) {
    case TPO_F32: loss_reduce<float>(L, w, B, N, M, mean != 0, loss, grid, s); break;
    case TPO_F64: loss_reduce<double>(L, w, B, N, M, mean != 0, loss, grid, s); break;
    case TPO_F16: loss_reduce<half_t>(L, w, B, N, M, mean != 0, loss, grid, s); break;
  }
  return check_launch("tpo_chamfer_loss_fwd");
}

extern "C" int tpo_chamfer_loss_bwd(int dtype, const void* xyz1, const void* xyz2,
                                    const int32_t* idx1, const int32_t* idx2,
                                    const void* grad_loss, int mean, int64_t B, int64_t N,
                                    int64_t M, void* gxyz1, void* gxyz2, void* stream) {
  if (B < 0 || N < 0 || M < 0 || B * (N + M) >= ((int64_t)1 << 40))
    return set_error(TPO_ERR_ARG, "tpo_chamfer_loss_bwd: bad sizes");
  if (B == 0 || (N == 0 && M == 0)) return TPO_OK;
  if (!grad_loss) return set_error(TPO_ERR_ARG, "tpo_chamfer_loss_bwd: null grad_loss");
  hipStream_t s = (hipStream_t)stream;
  const int64_t c1 = mean ? B * N : -1, c2 = mean ? B * M : -1;
  switch (dtype) {
    case TPO_F32: bwd_dispatch<float>(xyz1, xyz2, idx1, idx2, grad_loss, grad_loss, B, N, M, gxyz1, gxyz2, s, c1, c2); break;
    case TPO_F64: bwd_dispatch<double>(xyz1, xyz2, idx1, idx2, grad_loss, grad_loss, B, N, M, gxyz1, gxyz2, s, c1, c2); break;
    case TPO_F16: bwd_dispatch<half_t>(xyz1, xyz2, idx1, idx2, grad_loss, grad_loss, B, N, M, gxyz1, gxyz2, s, c1, c2); break;
    default: return set_error(TPO_ERR_DTYPE, "tpo_chamfer_loss_bwd: unsupported dtype %d", dtype);
  }
  return check_launch("tpo_chamfer_loss_bwd");
}
