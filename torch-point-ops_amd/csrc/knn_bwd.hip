// knn_bwd.hip -- KNN backward (replaces KNearestNeighborBackwardKernel and
// knn_cuda_backward, knn.cu:400-534).
//
// For query rows q < lengths1 and slots whose index is a reference (idx ==
// -1 padding skipped): diff = (2g)(p1 - p2) (norm 2) or g sign(p1 - p2)
// with sign 0 on equality (norm 1); grad_p1[q] += diff, grad_p2[idx] -=
// diff (knn.cu:436-462).
//
// grad_p2 is a scatter with ~K terms per reference point.  Scattered float
// atomics reach ~21 G/s on MI355X (one memory request per lane, whatever the
// scope), against ~300 G/s for atomics to consecutive addresses, so the
// scatter is done without them when the caller gives a workspace:
//  1. knn_bwd_entry_kernel, a lane per (query row, slot), 512 / K whole
//     rows of one cloud a workgroup: each lane computes its diff.  grad_p1 is
//     summed over the row's slots in slot order from LDS and written once
//     (zeros past lengths1).  Each term -diff goes into a record (reference
//     row within its bucket, -diff) and the workgroup groups its records by
//     bucket -- R consecutive reference rows of the cloud -- with an LDS
//     counting sort, into a region of its own, plus a table of (count,
//     start, largest |term|) per bucket.
//  2. knn_bwd_bucket_kernel, a workgroup per (cloud, bucket): it reads its
//     bucket's records from every entry workgroup of the cloud, adds them
//     into the bucket's rows in LDS in 64-bit fixed point (integer LDS
//     atomics; exact sums, the same bits on every run) and writes those rows
//     once (zeros where nothing lands): no zero fill, no global atomics.
// Without a workspace (or for D > 7, K > 512, or very long reference
// clouds) the terms go to a zero-filled grad_p2 by atomics: from the
// (row, slot) kernel for D <= 8, from a wave per row whose lanes run over
// the coordinates (consecutive addresses) otherwise.  Atomic and LDS
// accumulation orders are unspecified, as the reference's atomics are.
#include "knn_common.hpp"

#pragma clang fp contract(off)

namespace tpo {
namespace {

template <typename T>
__global__ __launch_bounds__(256) void bwd_fill_kernel(T* __restrict__ p, int64_t n, T v) {
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < n;
       t += (int64_t)gridDim.x * blockDim.x)
    p[t] = v;
}

unsigned bwd_grid_for(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 1 << 20) g = 1 << 20;
  return (unsigned)(g < 1 ? 1 : g);
}

template <typename T>
__device__ __forceinline__ T knn_bwd_diff(T g, T v1, T v2, int norm) {
  if (norm == 1) {
    const T sign = v1 > v2 ? (T)1 : (v1 == v2 ? (T)0 : (T)-1);
    return (T)(g * sign);
  }
  return (T)((T)((T)2 * g) * (T)(v1 - v2));
}

template <typename T>
struct BwdAcc {
  using type = float;
};
template <>
struct BwdAcc<double> {
  using type = double;
};

constexpr int KB1_THREADS = 512;   // entry kernel: (row, slot) lanes a workgroup
constexpr int KB2_THREADS = 1024;  // bucket kernel: a lane per entry workgroup
constexpr int KB_MAX_NB = 256;     // buckets a cloud at most
constexpr int KB_MIN_R = 512;      // reference rows a bucket at least
constexpr int KB_LDS2 = 49152;     // bytes of a bucket's rows in LDS at most

// Records: word 0 the reference row within the bucket (int bits), then -diff
// for each coordinate; 4 words for D <= 3, 8 for D <= 7.
__host__ __device__ inline int kb_record_words(int64_t D) { return D <= 3 ? 4 : 8; }

struct KbPlan {
  bool bucketed;
  int rpw, cpc, R, nb, rw;
  int64_t w1, rec_bytes, tab_bytes, total;
};

template <typename A>
KbPlan kb_plan(int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K) {
  KbPlan p{};
  p.bucketed = false;
  if (N <= 0 || P1 <= 0 || P2 <= 0 || D < 1 || D > 7 || K < 1 || K > KB1_THREADS) return p;
  p.rpw = KB1_THREADS / (int)K;
  const int64_t cpc = (P1 + p.rpw - 1) / p.rpw;
  int64_t R = (P2 + KB_MAX_NB - 1) / KB_MAX_NB;
  R = R < KB_MIN_R ? KB_MIN_R : ((R + 63) & ~(int64_t)63);
  if (R * D * 8 > KB_LDS2) return p;  // 64-bit accumulators
  if (N * cpc > 0x7fffffff || P1 * K > 0x7fffffff) return p;
  p.cpc = (int)cpc;
  p.R = (int)R;
  p.nb = (int)((P2 + R - 1) / R);
  p.rw = kb_record_words(D);
  p.w1 = N * cpc;
  auto al = [](int64_t x) { return (x + 255) & ~(int64_t)255; };
  p.rec_bytes = al(p.w1 * KB1_THREADS * p.rw * (int64_t)sizeof(A));
  p.tab_bytes = al(p.w1 * p.nb * (int64_t)sizeof(int4));
  p.total = p.rec_bytes + p.tab_bytes;
  p.bucketed = true;
  return p;
}

// Workgroup (cloud n, chunk c): rows [c rpw, min((c + 1) rpw, P1)) of cloud n,
// a lane per (row, slot).  BUCKETED: records + table (see the file header);
// otherwise the terms go straight to grad_p2 by atomics.
template <typename T, int DC, bool BUCKETED>
__global__ __launch_bounds__(KB1_THREADS) void knn_bwd_entry_kernel(
    const T* __restrict__ p1, const T* __restrict__ p2, const int64_t* __restrict__ len1,
    const int64_t* __restrict__ idxs, const T* __restrict__ gd, int norm, int P1, int P2,
    int D, int K, int rpw, int cpc, int R, int nb, T* __restrict__ gp1, T* __restrict__ gp2,
    typename BwdAcc<T>::type* __restrict__ rec, int4* __restrict__ tab) {
  using A = typename BwdAcc<T>::type;
  // diffs by (coordinate, row, slot), rows K + 1 apart (no bank conflicts
  // in the row sums)
  __shared__ T s_diff[DC * 2 * KB1_THREADS];
  __shared__ int s_cnt[BUCKETED ? KB_MAX_NB : 1];
  __shared__ unsigned s_max[BUCKETED ? KB_MAX_NB : 1];
  __shared__ int s_part[KB1_THREADS / 64];
  const int tid = threadIdx.x;
  const int n = blockIdx.x / cpc, c = blockIdx.x - n * cpc;
  const int q0 = c * rpw;
  const int nrow = min(rpw, P1 - q0);
  const int lr = tid / K, k = tid - lr * K;
  const int q = q0 + lr;
  int64_t l1 = len1[n];
  l1 = l1 < 0 ? 0 : (l1 > P1 ? P1 : l1);
  if (BUCKETED)
    for (int b = tid; b < nb; b += KB1_THREADS) {
      s_cnt[b] = 0;
      s_max[b] = 0u;
    }
  T diff[DC];
#pragma unroll
  for (int d = 0; d < DC; ++d) diff[d] = (T)0;
  int r = -1;
  if (lr < nrow && q < l1) {
    const int64_t slot = ((int64_t)n * P1 + q) * K + k;
    // the gradient and the query row do not depend on the index: load them
    // with it, so only the reference row waits for it
    const int64_t ri = idxs[slot];
    const T g = gd[slot];
    const T* __restrict__ a = p1 + ((int64_t)n * P1 + q) * D;
    T va[DC];
#pragma unroll
    for (int d = 0; d < DC; ++d) va[d] = d < D ? a[d] : (T)0;
    if (ri >= 0 && ri < P2) {  // -1 padding (knn.cu:439); other values are no reference
      r = (int)ri;
      const T* __restrict__ b = p2 + ((int64_t)n * P2 + r) * D;
#pragma unroll
      for (int d = 0; d < DC; ++d)
        if (d < D) diff[d] = knn_bwd_diff<T>(g, va[d], b[d], norm);
      if constexpr (!BUCKETED) {
        T* __restrict__ o = gp2 + ((int64_t)n * P2 + r) * D;
#pragma unroll
        for (int d = 0; d < DC; ++d)
          if (d < D) atomic_add(o + d, (T)(-diff[d]));
      }
    }
  }
  const int ks = K + 1;
#pragma unroll
  for (int d = 0; d < DC; ++d) s_diff[d * 2 * KB1_THREADS + lr * ks + k] = diff[d];
  __syncthreads();
  // grad_p1: a row's K diffs in slot order
  for (int e = tid; e < nrow * D; e += KB1_THREADS) {
    const int r2 = e / D, d = e - r2 * D;
    const T* __restrict__ col = s_diff + d * 2 * KB1_THREADS + r2 * ks;
    T sum = (T)0;
    for (int j = 0; j < K; ++j) sum = (T)(sum + col[j]);
    gp1[((int64_t)n * P1 + q0) * D + e] = sum;
  }
  if constexpr (BUCKETED) {
    // counting sort of this workgroup's records by bucket
    const int bk = r >= 0 ? r / R : -1;
    int rank = 0;
    if (bk >= 0) {
      rank = atomicAdd(&s_cnt[bk], 1);
      unsigned mbits = 0;  // largest |term| (as float bits: they order like the values)
#pragma unroll
      for (int d = 0; d < DC; ++d)
        if (d < D) mbits = max(mbits, __float_as_uint(__builtin_fabsf((float)diff[d])));
      atomicMax(&s_max[bk], mbits);
    }
    __syncthreads();
    // exclusive scan of the nb <= 256 counts, one a thread
    const int lane = tid & 63, w = tid >> 6;
    const int cnt = tid < nb ? s_cnt[tid] : 0;
    int incl = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o, 64);
      if (lane >= o) incl += v;
    }
    if (lane == 63) s_part[w] = incl;
    __syncthreads();
    int start = incl - cnt;
    for (int v = 0; v < w; ++v) start += s_part[v];
    // table [cloud][bucket][entry workgroup]: a bucket's entries are consecutive
    if (tid < nb)
      tab[((int64_t)n * nb + tid) * cpc + c] = make_int4(cnt, start, (int)s_max[tid], 0);
    __syncthreads();  // every count read before the starts overwrite them
    if (tid < nb) s_cnt[tid] = start;
    __syncthreads();
    if (bk >= 0) {
      const int rw = kb_record_words(D);
      A* __restrict__ o = rec + ((int64_t)blockIdx.x * KB1_THREADS + s_cnt[bk] + rank) * rw;
      if constexpr (sizeof(A) == 4) {
        if (rw == 4) {
          *reinterpret_cast<float4*>(o) = make_float4(__int_as_float(r - bk * R), (float)-diff[0],
                                                      D > 1 ? (float)-diff[1] : 0.f,
                                                      D > 2 ? (float)-diff[2] : 0.f);
          return;
        }
        o[0] = __int_as_float(r - bk * R);
      } else {
        o[0] = __longlong_as_double((long long)(r - bk * R));
      }
#pragma unroll
      for (int d = 0; d < DC; ++d)
        if (d < D) o[1 + d] = (A)-diff[d];
    }
  }
}

// Reads the records of (cloud n, bucket j) -- L lanes per entry workgroup
// (every thread busy when the cloud has KB2_THREADS / L of them), each taking
// every L-th group of U records, U in flight -- and calls f(row, v) for each
// (v: its D terms).
template <typename A, typename F>
__device__ __forceinline__ void kb_for_records(const A* __restrict__ rec,
                                               const int4* __restrict__ t, int n, int cpc, int D,
                                               F&& f) {
  const int rw = kb_record_words(D);
  const int L = cpc * 4 <= KB2_THREADS ? 4 : (cpc * 2 <= KB2_THREADS ? 2 : 1);
  const int sub = (int)threadIdx.x % L;
  constexpr int U = 4;
  for (int c = (int)threadIdx.x / L; c < cpc; c += KB2_THREADS / L) {
    const int4 cs = t[c];
    const A* __restrict__ src = rec + ((int64_t)(n * cpc + c) * KB1_THREADS + cs.y) * rw;
    for (int i0 = sub * U; i0 < cs.x; i0 += L * U) {
      int row[U];
      A v[U][7];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        row[u] = -1;
        if (i0 + u < cs.x) {
          const A* __restrict__ x = src + (int64_t)(i0 + u) * rw;
          if constexpr (sizeof(A) == 4) {
            if (rw == 4) {
              const float4 q = *reinterpret_cast<const float4*>(x);
              row[u] = __float_as_int(q.x);
              v[u][0] = q.y;
              v[u][1] = q.z;
              v[u][2] = q.w;
            } else {
              row[u] = __float_as_int(x[0]);
#pragma unroll
              for (int d = 0; d < 7; ++d) v[u][d] = d < D ? x[1 + d] : (A)0;
            }
          } else {
            row[u] = (int)__double_as_longlong(x[0]);
#pragma unroll
            for (int d = 0; d < 7; ++d) v[u][d] = d < D ? x[1 + d] : (A)0;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (row[u] >= 0) f(row[u], v[u]);
    }
  }
}

// Workgroup (cloud n, bucket j): rows [j R, min((j + 1) R, P2)) of cloud n's
// grad_p2, from the records of the cloud's cpc entry workgroups, summed in
// 64-bit fixed point with integer LDS atomics (float LDS atomics run about
// 25 times slower here than integer ones).  The scale puts the bucket's
// largest |term| (from the entry workgroups' table) below 2^52, lower when
// the bucket holds more than 2^11 records, so that no row sum can leave the
// int64 range; each term is rounded to nearest on conversion (exact for
// float terms within ~2^28 of the largest).  Integer sums are exact and
// order-free, so grad_p2 is the same on every run; each row is converted
// back once.
template <typename T>
__global__ __launch_bounds__(KB2_THREADS) void knn_bwd_bucket_kernel(
    const typename BwdAcc<T>::type* __restrict__ rec, const int4* __restrict__ tab, int P2, int D,
    int cpc, int R, int nb, T* __restrict__ gp2) {
  using A = typename BwdAcc<T>::type;
  extern __shared__ __align__(16) char s_dyn[];
  unsigned long long* __restrict__ acc = reinterpret_cast<unsigned long long*>(s_dyn);
  __shared__ unsigned s_max, s_total;
  const int tid = threadIdx.x;
  const int n = blockIdx.x / nb, j = blockIdx.x - n * nb;
  const int r0 = j * R, ns = min(R, P2 - r0);
  for (int e = tid; e < ns * D; e += KB2_THREADS) acc[e] = 0ull;
  if (tid == 0) s_max = s_total = 0u;
  __syncthreads();
  const int4* __restrict__ t = tab + ((int64_t)n * nb + j) * cpc;
  // records in the bucket (no row takes more terms) and the largest |term|
  unsigned tot = 0, m = 0;
  for (int c = tid; c < cpc; c += KB2_THREADS) {
    const int4 cs = t[c];
    tot += (unsigned)cs.x;
    m = max(m, (unsigned)cs.z);
  }
  for (int o = 32; o > 0; o >>= 1) {
    tot += (unsigned)__shfl_xor((int)tot, o, 64);
    m = max(m, (unsigned)__shfl_xor((int)m, o, 64));
  }
  if ((tid & 63) == 0 && tot) {
    atomicAdd(&s_total, tot);
    atomicMax(&s_max, m);
  }
  __syncthreads();
  const unsigned mb = s_max, total = s_total;
  // 2^S puts the largest term below 2^(top + 1), top = min(51, 62 - ceil(log2
  // total)): S = top - floor(log2 max) (float bits of a normal: exponent
  // field - 127; a subnormal maximum counts as 2^-126, which only drops bits
  // below 2^-178)
  const int e2 = (int)((mb >> 23) & 0xff) - 127;
  const int lg = total > 1u ? 32 - __builtin_clz(total - 1u) : 0;
  const int S = min(51, 62 - lg) - (e2 < -126 ? -126 : e2);
  T* __restrict__ o = gp2 + ((int64_t)n * P2 + r0) * D;
  if (mb < 0x7f800000u) {
    if (mb != 0u) {
      const double scale = __builtin_ldexp(1.0, S);
      kb_for_records<A>(rec, t, n, cpc, D, [&](int row, const A (&v)[7]) {
#pragma unroll
        for (int d = 0; d < 7; ++d)
          if (d < D)
            atomicAdd(acc + row * D + d,
                      (unsigned long long)(long long)__builtin_rint((double)v[d] * scale));
      });
    }
    __syncthreads();
    const double inv = __builtin_ldexp(1.0, -S);
    for (int e = tid; e < ns * D; e += KB2_THREADS) o[e] = (T)((double)(long long)acc[e] * inv);
  } else {  // an infinite or NaN term: the sums in floating point (order unspecified)
    A* __restrict__ fa = reinterpret_cast<A*>(s_dyn);
    for (int e = tid; e < ns * D; e += KB2_THREADS) fa[e] = (A)0;
    __syncthreads();
    kb_for_records<A>(rec, t, n, cpc, D, [&](int row, const A (&v)[7]) {
#pragma unroll
      for (int d = 0; d < 7; ++d)
        if (d < D) atomicAdd(fa + row * D + d, v[d]);
    });
    __syncthreads();
    for (int e = tid; e < ns * D; e += KB2_THREADS) o[e] = (T)fa[e];
  }
}

// Any D and K: one wave per query row, lanes over the coordinates (64 at a
// time), slots in order; the row's index and gradient are wave-uniform, the
// p2 row loads and grad_p2 atomics of a wave are consecutive.
template <typename T>
__global__ __launch_bounds__(256) void knn_bwd_rows_kernel(
    const T* __restrict__ p1, const T* __restrict__ p2, const int64_t* __restrict__ len1,
    const int64_t* __restrict__ idxs, const T* __restrict__ gd, int norm, int64_t rows,
    int64_t P1, int64_t P2, int64_t D, int64_t K, T* __restrict__ gp1, T* __restrict__ gp2) {
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * 4 + wave_id();
  if (row >= rows) return;
  const int64_t n = row / P1, q = row - n * P1;
  const bool active = q < len1[n];
  for (int64_t d0 = 0; d0 < D; d0 += 64) {
    const int64_t d = d0 + lane;
    const bool dv = d < D;
    T acc = (T)0;
    if (active) {
      const T v1 = dv ? p1[row * D + d] : (T)0;
      for (int64_t k = 0; k < K; ++k) {
        const int64_t r = idxs[row * K + k];
        if (r < 0 || r >= P2) continue;
        const T g = gd[row * K + k];
        if (dv) {
          const T df = knn_bwd_diff<T>(g, v1, p2[(n * P2 + r) * D + d], norm);
          acc = (T)(acc + df);
          atomic_add(gp2 + (n * P2 + r) * D + d, (T)(-df));
        }
      }
    }
    if (dv) gp1[row * D + d] = acc;
  }
}

template <typename T>
int64_t bwd_workspace(int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K) {
  const KbPlan p = kb_plan<typename BwdAcc<T>::type>(N, P1, P2, D, K);
  return p.bucketed ? p.total : 0;
}

template <typename T>
void launch_bwd(const void* p1, const void* p2, const int64_t* l1, const int64_t* idxs,
                const void* gd, int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K, int norm,
                void* gp1, void* gp2, void* ws, int64_t ws_bytes, hipStream_t s) {
  using A = typename BwdAcc<T>::type;
  const int64_t rows = N * P1;
  if (K == 0) {  // no slots: both gradients are zero
    if (rows * D > 0)
      hipLaunchKernelGGL(bwd_fill_kernel<T>, dim3(bwd_grid_for(rows * D)), dim3(256), 0, s,
                         (T*)gp1, rows * D, (T)0);
    if (N * P2 * D > 0)
      hipLaunchKernelGGL(bwd_fill_kernel<T>, dim3(bwd_grid_for(N * P2 * D)), dim3(256), 0, s,
                         (T*)gp2, N * P2 * D, (T)0);
    return;
  }
  const KbPlan p = kb_plan<A>(N, P1, P2, D, K);
  if (p.bucketed && ws && ws_bytes >= p.total) {
    A* rec = reinterpret_cast<A*>(ws);
    int4* tab = reinterpret_cast<int4*>((char*)ws + p.rec_bytes);
    if (D <= 4)
      hipLaunchKernelGGL((knn_bwd_entry_kernel<T, 4, true>), dim3((unsigned)p.w1),
                         dim3(KB1_THREADS), 0, s, (const T*)p1, (const T*)p2, l1, idxs,
                         (const T*)gd, norm, (int)P1, (int)P2, (int)D, (int)K, p.rpw, p.cpc, p.R,
                         p.nb, (T*)gp1, (T*)gp2, rec, tab);
    else
      hipLaunchKernelGGL((knn_bwd_entry_kernel<T, 8, true>), dim3((unsigned)p.w1),
                         dim3(KB1_THREADS), 0, s, (const T*)p1, (const T*)p2, l1, idxs,
                         (const T*)gd, norm, (int)P1, (int)P2, (int)D, (int)K, p.rpw, p.cpc, p.R,
                         p.nb, (T*)gp1, (T*)gp2, rec, tab);
    hipLaunchKernelGGL(knn_bwd_bucket_kernel<T>, dim3((unsigned)(N * p.nb)), dim3(KB2_THREADS),
                       (size_t)p.R * D * 8, s, (const A*)rec, (const int4*)tab, (int)P2,
                       (int)D, p.cpc, p.R, p.nb, (T*)gp2);
    return;
  }
  if (N * P2 * D > 0)
    hipLaunchKernelGGL(bwd_fill_kernel<T>, dim3(bwd_grid_for(N * P2 * D)), dim3(256), 0, s,
                       (T*)gp2, N * P2 * D, (T)0);
  if (rows == 0) return;
  if (D <= 8 && K <= KB1_THREADS && P1 <= 0x7fffffff && P2 <= 0x7fffffff &&
      N * ((P1 + KB1_THREADS / K - 1) / (KB1_THREADS / K)) <= 0x7fffffff) {
    const int rpw = KB1_THREADS / (int)K;
    const int cpc = (int)((P1 + rpw - 1) / rpw);
    if (D <= 4)
      hipLaunchKernelGGL((knn_bwd_entry_kernel<T, 4, false>), dim3((unsigned)(N * cpc)),
                         dim3(KB1_THREADS), 0, s, (const T*)p1, (const T*)p2, l1, idxs,
                         (const T*)gd, norm, (int)P1, (int)P2, (int)D, (int)K, rpw, cpc, 1, 1,
                         (T*)gp1, (T*)gp2, (A*)nullptr, (int4*)nullptr);
    else
      hipLaunchKernelGGL((knn_bwd_entry_kernel<T, 8, false>), dim3((unsigned)(N * cpc)),
                         dim3(KB1_THREADS), 0, s, (const T*)p1, (const T*)p2, l1, idxs,
                         (const T*)gd, norm, (int)P1, (int)P2, (int)D, (int)K, rpw, cpc, 1, 1,
                         (T*)gp1, (T*)gp2, (A*)nullptr, (int4*)nullptr);
    return;
  }
  hipLaunchKernelGGL(knn_bwd_rows_kernel<T>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s,
                     (const T*)p1, (const T*)p2, l1, idxs, (const T*)gd, norm, rows, P1, P2, D,
                     K, (T*)gp1, (T*)gp2);
}

}  // namespace
}  // namespace tpo

using namespace tpo;

extern "C" int64_t tpo_knn_bwd_workspace_size(int dtype, int64_t N, int64_t P1, int64_t P2,
                                              int64_t D, int64_t K) {
  switch (dtype) {
    case TPO_F32: return bwd_workspace<float>(N, P1, P2, D, K);
    case TPO_F64: return bwd_workspace<double>(N, P1, P2, D, K);
    case TPO_F16: return bwd_workspace<half_t>(N, P1, P2, D, K);
    default: return 0;
  }
}

extern "C" int tpo_knn_bwd_ws(int dtype, const void* p1, const void* p2, const int64_t* lengths1,
                              const int64_t* lengths2, const int64_t* idxs, int norm,
                              const void* grad_dists, int64_t N, int64_t P1, int64_t P2, int64_t D,
                              int64_t K, void* grad_p1, void* grad_p2, void* workspace,
                              int64_t workspace_bytes, void* stream) {
  (void)lengths2;
  if (N < 0 || P1 < 0 || P2 < 0 || D < 1 || K < 0)
    return set_error(TPO_ERR_ARG, "tpo_knn_bwd: bad sizes");
  if (norm != 1 && norm != 2) return set_error(TPO_ERR_ARG, "Norm must be 1 or 2.");
  if (workspace_bytes < 0) return set_error(TPO_ERR_ARG, "tpo_knn_bwd: bad workspace size");
  if (N == 0 || (P1 == 0 && P2 == 0)) return TPO_OK;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case TPO_F32: launch_bwd<float>(p1, p2, lengths1, idxs, grad_dists, N, P1, P2, D, K, norm, grad_p1, grad_p2, workspace, workspace_bytes, s); break;
    case TPO_F64: launch_bwd<double>(p1, p2, lengths1, idxs, grad_dists, N, P1, P2, D, K, norm, grad_p1, grad_p2, workspace, workspace_bytes, s); break;
    case TPO_F16: launch_bwd<half_t>(p1, p2, lengths1, idxs, grad_dists, N, P1, P2, D, K, norm, grad_p1, grad_p2, workspace, workspace_bytes, s); break;
    default: return set_error(TPO_ERR_DTYPE, "tpo_knn_bwd: unsupported dtype %d", dtype);
  }
  return check_launch("tpo_knn_bwd");
}

extern "C" int tpo_knn_bwd(int dtype, const void* p1, const void* p2, const int64_t* lengths1,
                           const int64_t* lengths2, const int64_t* idxs, int norm,
                           const void* grad_dists, int64_t N, int64_t P1, int64_t P2, int64_t D,
                           int64_t K, void* grad_p1, void* grad_p2, void* stream) {
  return tpo_knn_bwd_ws(dtype, p1, p2, lengths1, lengths2, idxs, norm, grad_dists, N, P1, P2, D,
                        K, grad_p1, grad_p2, nullptr, 0, stream);
}
