// chamfer.hip -- Chamfer distance forward/backward for gfx950.
//
// Forward (replaces chamfer_dist_kernel, chamfer.cu:36-167).
//   One launch covers both directions.  A workgroup owns 64*Q query points
//   (Q per lane, held in VGPRs) of one (direction, cloud) and its 4 waves split
//   the reference cloud into 4 contiguous chunks.  Each wave streams its chunk
//   through SGPRs (wave-uniform scalar loads, no LDS traffic in the hot loop),
//   so the inner loop is 6 VALU ops per pair (3 sub, mul, 2 fma) plus half a
//   v_min3 for the running minimum.
//   First-index argmin without per-pair index bookkeeping: per tile of 16
//   references keep only the tile minimum; a tile replaces the running best
//   only when strictly smaller (so the earliest tile holding the minimum wins);
//   at the end the winning tile is re-scanned with the identical formula and
//   the first position whose distance equals the minimum bit-for-bit is the
//   index.  Chunks merge in LDS in index order with strict-less, so ties go to
//   the lowest index -- the reference's rule (chamfer.cu:69-72, 159-162).
// Backward (replaces chamfer_dist_grad_kernel, chamfer.cu:200-234).
//   grad_q[i] = 2 g_i (q_i - r_idx[i]) - sum over the other cloud's points j
//   matched to i of 2 g_j (r_j - q_i).  When one cloud's gradient fits in LDS
//   (<= 12288 points, float/half) a 1024-thread workgroup per (cloud, batch)
//   accumulates the scattered terms with LDS atomics, adds its points' direct
//   terms and writes every element once: no global atomics, no zero-fill.
//   (float16: terms are computed in half like the reference, accumulated in
//   float and rounded once.)  Otherwise pass 1 stores the direct terms (which
//   initialises both outputs) and pass 2 scatters the negated terms with
//   hardware atomics, like the reference.
#include <stdio.h>

#include "tpo_common.hpp"

#pragma clang fp contract(off)

namespace tpo {

constexpr int CH_WAVES = 4;
constexpr int CH_TILE = 16;

// Copy a wave-uniform (SGPR) value into a VGPR.  On gfx950 a VALU op with an
// SGPR source issues at 4 cycles per wave64 instruction, while VGPR-only
// FP32 ops issue at ~2.3-2.7; one v_mov per reference coordinate, shared by
// the Q queries of the lane, lets every subtraction use VGPR operands.
__device__ __forceinline__ float to_vgpr(float s) {
  float v;
  asm("v_mov_b32 %0, %1" : "=v"(v) : "s"(s));
  return v;
}
__device__ __forceinline__ double to_vgpr(double s) { return s; }
__device__ __forceinline__ half_t to_vgpr(half_t s) { return s; }

__device__ __forceinline__ float vmin(float a, float b) { return __builtin_fminf(a, b); }
__device__ __forceinline__ double vmin(double a, double b) { return __builtin_fmin(a, b); }
__device__ __forceinline__ half_t vmin(half_t a, half_t b) { return __builtin_fminf16(a, b); }

template <typename T, int Q>
__global__ __launch_bounds__(256) void chamfer_fwd_kernel(
    const T* __restrict__ xyz1, const T* __restrict__ xyz2, int B, int N, int M, int nqb1,
    int nqb2, T* __restrict__ dist1, T* __restrict__ dist2, int32_t* __restrict__ idx1,
    int32_t* __restrict__ idx2) {
  __shared__ T s_d[CH_WAVES][64 * Q];
  __shared__ int s_i[CH_WAVES][64 * Q];

  int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int g1 = B * nqb1;
  const int dir = lb >= g1;
  if (dir) lb -= g1;
  const int nqb = dir ? nqb2 : nqb1;
  const int b = lb / nqb;
  const int qb = lb - b * nqb;
  const int nq = dir ? M : N;
  const int nr = dir ? N : M;
  const T* __restrict__ qp = (dir ? xyz2 : xyz1) + (size_t)b * nq * 3;
  const T* __restrict__ rp = (dir ? xyz1 : xyz2) + (size_t)b * nr * 3;

  const int w = wave_id(), lane = lane_id();
  const int chunk = ((nr + CH_WAVES * CH_TILE - 1) / (CH_WAVES * CH_TILE)) * CH_TILE;
  const int c0 = w * chunk;
  const int c1 = min(nr, c0 + chunk);

  T qx[Q], qy[Q], qz[Q], best[Q];
  int bt[Q];
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    int gq = qb * 64 * Q + i * 64 + lane;
    gq = gq < nq ? gq : nq - 1;
    qx[i] = qp[3 * gq];
    qy[i] = qp[3 * gq + 1];
    qz[i] = qp[3 * gq + 2];
    best[i] = Lim<T>::inf();
    bt[i] = c0;
  }

  int t0 = c0;
  for (; t0 + CH_TILE <= c1; t0 += CH_TILE) {
    T tmin[Q];
#pragma unroll
    for (int i = 0; i < Q; ++i) tmin[i] = Lim<T>::inf();
    const T* __restrict__ r = rp + 3 * t0;
#pragma unroll
    for (int j = 0; j < CH_TILE; ++j) {
      const T rx = to_vgpr(r[3 * j]), ry = to_vgpr(r[3 * j + 1]), rz = to_vgpr(r[3 * j + 2]);
#pragma unroll
      for (int i = 0; i < Q; ++i)
        tmin[i] = vmin(tmin[i], sq3((T)(rx - qx[i]), (T)(ry - qy[i]), (T)(rz - qz[i])));
    }
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const bool lt = tmin[i] < best[i];
      best[i] = lt ? tmin[i] : best[i];
      bt[i] = lt ? t0 : bt[i];
    }
  }
  if (t0 < c1) {  // partial last tile of this chunk
    T tmin[Q];
#pragma unroll
    for (int i = 0; i < Q; ++i) tmin[i] = Lim<T>::inf();
    for (int j = t0; j < c1; ++j) {
      const T rx = rp[3 * j], ry = rp[3 * j + 1], rz = rp[3 * j + 2];
#pragma unroll
      for (int i = 0; i < Q; ++i)
        tmin[i] = vmin(tmin[i], sq3((T)(rx - qx[i]), (T)(ry - qy[i]), (T)(rz - qz[i])));
    }
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const bool lt = tmin[i] < best[i];
      best[i] = lt ? tmin[i] : best[i];
      bt[i] = lt ? t0 : bt[i];
    }
  }

  // Recover the first index inside the winning tile (same formula, same bits).
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    int found = 0x7fffffff;
    if (c0 < c1) {
      const int tb = bt[i];
      for (int k = 0; k < CH_TILE; ++k) {
        const int j = tb + k;
        if (j < c1 && found == 0x7fffffff) {
          const T d = sq3((T)(rp[3 * j] - qx[i]), (T)(rp[3 * j + 1] - qy[i]),
                          (T)(rp[3 * j + 2] - qz[i]));
          if (d == best[i]) found = j;
        }
      }
      if (found == 0x7fffffff) found = c0;  // all-NaN chunk: keep its first index
    }
    s_d[w][i * 64 + lane] = best[i];
    s_i[w][i * 64 + lane] = found;
  }
  __syncthreads();

  T* __restrict__ dout = (dir ? dist2 : dist1) + (size_t)b * nq;
  int32_t* __restrict__ iout = (dir ? idx2 : idx1) + (size_t)b * nq;
  for (int e = threadIdx.x; e < 64 * Q; e += 256) {
    const int gq = qb * 64 * Q + e;
    if (gq >= nq) continue;
    T bd = s_d[0][e];
    int bi = s_i[0][e];
#pragma unroll
    for (int v = 1; v < CH_WAVES; ++v) {
      const T d = s_d[v][e];
      if (d < bd) {
        bd = d;
        bi = s_i[v][e];
      }
    }
    if (bi == 0x7fffffff) {  // empty reference cloud: zeros, as the reference's init
      bd = (T)0;
      bi = 0;
    }
    dout[gq] = bd;
    iout[gq] = bi;
  }
}

// ---------------------------------------------------------------- backward
// Pass 1: grad_q[i] = g (q_i - r_idx[i]) with g = 2 grad_dist[i] (in dtype);
// every element of both outputs is written here.
template <typename T>
__global__ __launch_bounds__(256) void chamfer_bwd_direct_kernel(
    const T* __restrict__ xyz1, const T* __restrict__ xyz2, const int32_t* __restrict__ idx1,
    const int32_t* __restrict__ idx2, const T* __restrict__ gd1, const T* __restrict__ gd2,
    int64_t B, int64_t N, int64_t M, T* __restrict__ g1, T* __restrict__ g2) {
  const int64_t n1 = B * N, total = n1 + B * M;
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
      const T g = (T)((dir ? gd2 : gd1)[u] * (T)2);
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
    const int32_t* __restrict__ idx2, const T* __restrict__ gd1, const T* __restrict__ gd2,
    int64_t B, int64_t N, int64_t M, T* __restrict__ g1, T* __restrict__ g2) {
  const int64_t n1 = B * N, total = n1 + B * M;
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
    const T g = (T)((dir ? gd2 : gd1)[u] * (T)2);
    const int64_t ro = (b * nr + j2) * 3;
    atomic_add(gr + ro, (T)(-(T)(g * (T)(q[3 * u] - r[ro]))));
    atomic_add(gr + ro + 1, (T)(-(T)(g * (T)(q[3 * u + 1] - r[ro + 1]))));
    atomic_add(gr + ro + 2, (T)(-(T)(g * (T)(q[3 * u + 2] - r[ro + 2]))));
  }
}

constexpr int CH_BWD_LDS_FLOATS = 36864;  // 144 KiB: 12288 points x 3

template <typename T>
__global__ __launch_bounds__(1024) void chamfer_bwd_fused_kernel(
    const T* __restrict__ xyz1, const T* __restrict__ xyz2, const int32_t* __restrict__ idx1,
    const int32_t* __restrict__ idx2, const T* __restrict__ gd1, const T* __restrict__ gd2, int N,
    int M, T* __restrict__ g1, T* __restrict__ g2) {
  __shared__ float acc[CH_BWD_LDS_FLOATS];
  const int c = blockIdx.x & 1;  // 0: gradient of cloud 1, 1: of cloud 2
  const int b = blockIdx.x >> 1;
  const int n_own = c ? M : N, n_oth = c ? N : M;
  const T* __restrict__ own = (c ? xyz2 : xyz1) + (size_t)b * n_own * 3;
  const T* __restrict__ oth = (c ? xyz1 : xyz2) + (size_t)b * n_oth * 3;
  const int32_t* __restrict__ idx_own = (c ? idx2 : idx1) + (size_t)b * n_own;
  const int32_t* __restrict__ idx_oth = (c ? idx1 : idx2) + (size_t)b * n_oth;
  const T* __restrict__ gd_own = (c ? gd2 : gd1) + (size_t)b * n_own;
  const T* __restrict__ gd_oth = (c ? gd1 : gd2) + (size_t)b * n_oth;
  T* __restrict__ out = (c ? g2 : g1) + (size_t)b * n_own * 3;

  for (int i = threadIdx.x; i < 3 * n_own; i += 1024) acc[i] = 0.f;
  __syncthreads();
  // other cloud's points j whose nearest point is i (chamfer.cu:229-231 of
  // the other direction): acc[i] += -(g_j (r_j - q_i))
  for (int j = threadIdx.x; j < n_oth; j += 1024) {
    const int i = idx_oth[j];
    if (i < 0 || i >= n_own) continue;
    const T g = (T)(gd_oth[j] * (T)2);
#pragma unroll
    for (int k = 0; k < 3; ++k)
      atomicAdd(&acc[3 * i + k], -(float)(T)(g * (T)(oth[3 * j + k] - own[3 * i + k])));
  }
  __syncthreads();
  // direct term of the own points (chamfer.cu:226-228)
  for (int i = threadIdx.x; i < n_own; i += 1024) {
    const int j2 = idx_own[i];
    const bool ok = j2 >= 0 && j2 < n_oth;
    const T g = (T)(gd_own[i] * (T)2);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const T d = ok ? (T)(g * (T)(own[3 * i + k] - oth[3 * j2 + k])) : (T)0;
      out[3 * i + k] = (T)(acc[3 * i + k] + (float)d);
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

template <typename T>
static void fwd_dispatch(const void* x1, const void* x2, int B, int N, int M, void* d1, void* d2,
                         int32_t* i1, int32_t* i2, hipStream_t s) {
  // Largest per-lane query count that still gives >= 2 workgroups per CU.
  const int64_t q = (int64_t)B * ((int64_t)N + M);
  if (q >= (int64_t)512 * 64 * 8) launch_fwd<T, 8>(x1, x2, B, N, M, d1, d2, i1, i2, s);
  else if (q >= (int64_t)512 * 64 * 4) launch_fwd<T, 4>(x1, x2, B, N, M, d1, d2, i1, i2, s);
  else if (q >= (int64_t)512 * 64 * 2) launch_fwd<T, 2>(x1, x2, B, N, M, d1, d2, i1, i2, s);
  else launch_fwd<T, 1>(x1, x2, B, N, M, d1, d2, i1, i2, s);
}

template <typename T>
static void bwd_dispatch(const void* x1, const void* x2, const int32_t* i1, const int32_t* i2,
                         const void* gd1, const void* gd2, int64_t B, int64_t N, int64_t M,
                         void* g1, void* g2, hipStream_t s) {
  const int64_t total = B * (N + M);
  if (total == 0) return;
  if (sizeof(T) <= 4 && 3 * std::max(N, M) <= CH_BWD_LDS_FLOATS && 2 * B < (1 << 30)) {
    hipLaunchKernelGGL(chamfer_bwd_fused_kernel<T>, dim3((unsigned)(2 * B)), dim3(1024), 0, s,
                       (const T*)x1, (const T*)x2, i1, i2, (const T*)gd1, (const T*)gd2, (int)N,
                       (int)M, (T*)g1, (T*)g2);
    return;
  }
  const int64_t blocks = std::min<int64_t>((total + 255) / 256, 65536);
  hipLaunchKernelGGL(chamfer_bwd_direct_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, s,
                     (const T*)x1, (const T*)x2, i1, i2, (const T*)gd1, (const T*)gd2, B, N, M,
                     (T*)g1, (T*)g2);
  hipLaunchKernelGGL(chamfer_bwd_scatter_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, s,
                     (const T*)x1, (const T*)x2, i1, i2, (const T*)gd1, (const T*)gd2, B, N, M,
                     (T*)g1, (T*)g2);
}

}  // namespace tpo

using namespace tpo;

extern "C" int tpo_chamfer_fwd(int dtype, const void* xyz1, const void* xyz2, int64_t B,
                               int64_t N, int64_t M, void* dist1, void* dist2, int32_t* idx1,
                               int32_t* idx2, void* stream) {
  if (B < 0 || N < 0 || M < 0 || N >= (1 << 28) || M >= (1 << 28) ||
      B * (N + M) >= ((int64_t)1 << 31))
    return set_error(TPO_ERR_ARG, "tpo_chamfer_fwd: bad sizes B=%lld N=%lld M=%lld",
                     (long long)B, (long long)N, (long long)M);
  if (B == 0 || (N == 0 && M == 0)) return TPO_OK;
  if ((N > 0 && (!xyz1 || !dist1 || !idx1)) || (M > 0 && (!xyz2 || !dist2 || !idx2)))
    return set_error(TPO_ERR_ARG, "tpo_chamfer_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case TPO_F32: fwd_dispatch<float>(xyz1, xyz2, (int)B, (int)N, (int)M, dist1, dist2, idx1, idx2, s); break;
    case TPO_F64: fwd_dispatch<double>(xyz1, xyz2, (int)B, (int)N, (int)M, dist1, dist2, idx1, idx2, s); break;
    case TPO_F16: fwd_dispatch<half_t>(xyz1, xyz2, (int)B, (int)N, (int)M, dist1, dist2, idx1, idx2, s); break;
    default: return set_error(TPO_ERR_DTYPE, "tpo_chamfer_fwd: unsupported dtype %d", dtype);
  }
  return check_launch("tpo_chamfer_fwd");
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
