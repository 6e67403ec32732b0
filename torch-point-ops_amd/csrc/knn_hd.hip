// knn_hd.hip -- exact K nearest neighbours of float points of 64 or 128
// dimensions against long reference clouds with few queries (config 5's
// shape in float: the reference's KNearestNeighborKernelV0, knn.cu:16-60,
// MinK slot layout of mink.cuh:77-121), references sliced over the GPU.
#include <utility>

#include "knn_common.hpp"

#pragma clang fp contract(off)

namespace tpo {
namespace {

// A long reference cloud and few queries (config 5's shape in float: 16384
// queries, 65536 references of 128 dimensions) leave most of the GPU idle
// with one lane per query.  The references [K, lengths2) are cut into S
// slices, and a workgroup per (cloud, 256 queries, slice) runs its own MinK
// seeded with the K fill references (0 .. K-1) over its slice only.  That
// local MinK keeps the K smallest values of a subset of every prefix the
// real process has seen, so its threshold is never below the real one: every
// reference the real process inserts is inserted locally too, and the local
// insertions (distance, index) of a slice are a superset of the real ones.
// The merge replays MinK over the fill and the slices' candidates in index
// order; a candidate that is no real insertion fails the replay's test (the
// replay's state equals the real state at every real insertion), so the
// slot layout and values are the single sequential pass's, bit for bit.  A
// slice with more than HD_CAP candidates is recomputed by the merge.
//
// Reference points reach the lanes through DPP: each 16-lane row of the wave
// loads the same reference row with ordinary vector loads (lane k of a row:
// dimensions 64g + 4k .. + 3), issued HD_J references ahead, and
// dimension 64g + 4k + e enters the subtraction as VGPR (g, e) of lane k
// broadcast over its row (row_newbcast:k, folded into v_sub_f32_dpp), so a
// dimension costs one subtraction and one FMA and nothing waits on scalar
// loads.  Every lane of a wave that has a query takes part (lanes past
// lengths1 or P1 compute on zeros and never insert).  Candidates are found
// per chunk of 32 references: the chunk's distances go to LDS and into a mask
// against the lane's threshold; each lane then walks its own candidates in
// order against the updated threshold, so the wave pays the O(K) slot update
// max-over-lanes(candidates per chunk) times.
constexpr int HD_CAP = 256;  // candidates kept per (query, slice); a multiple of 16
constexpr int HD_J = 4;      // references per load step

template <int E>
__device__ __forceinline__ float f4_at(const float4& v) {
  if constexpr (E == 0) return v.x;
  else if constexpr (E == 1) return v.y;
  else if constexpr (E == 2) return v.z;
  else return v.w;
}
// knn.cu:148-158 over dimensions 0 .. DT-1 in order; dimension d of the
// reference is lane (d % 64) / 4 of the row, VGPR (d / 64, d % 4)
template <int NORM, int DT, int... D>
__device__ __forceinline__ float hd_dist(const float (&qr)[DT], const float4 (&rv)[DT / 64],
                                         std::integer_sequence<int, D...>) {
  float acc = 0.f;
  ((acc = NORM == 2
              ? knn_acc2(acc, qr[D] - row_bcast<(D % 64) / 4>(f4_at<D % 4>(rv[D / 64])), D == 0)
              : knn_acc1(acc, qr[D] - row_bcast<(D % 64) / 4>(f4_at<D % 4>(rv[D / 64])), D == 0)),
   ...);
  return acc;
}

// the same distance with both points read from memory (float4 steps)
template <int NORM, int DT>
__device__ __forceinline__ float hd_dist_mem(const float4* __restrict__ q, const float4* __restrict__ r) {
  float acc = 0.f;
#pragma unroll 4
  for (int v = 0; v < DT / 4; ++v) {
    const float4 a = q[v], b = r[v];
    const float x[4] = {a.x - b.x, a.y - b.y, a.z - b.z, a.w - b.w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      acc = NORM == 2 ? knn_acc2(acc, x[e], v == 0 && e == 0) : knn_acc1(acc, x[e], v == 0 && e == 0);
  }
  return acc;
}

// workspace: per (row, slice) the candidate count, distances and indices;
// per row the K fill distances (written by the first slice's workgroups)
struct HdLayout {
  int64_t cnt, dist, idx, fill, total;
};
HdLayout hd_layout(int64_t rows, int64_t S, int64_t K) {
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  HdLayout L;
  L.cnt = 0;
  L.dist = up(rows * S * 4);
  L.idx = L.dist + up(rows * S * HD_CAP * 4);
  L.fill = L.idx + up(rows * S * HD_CAP * 4);
  L.total = L.fill + up(rows * K * 4);
  return L;
}

template <int DT, int NORM, int KC>
__global__ __launch_bounds__(256) void knn_hd_slice_kernel(
    const float* __restrict__ p1, const float* __restrict__ p2, const int64_t* __restrict__ len1,
    const int64_t* __restrict__ len2, int P1, int P2, int K, int nqb, int S, int slen,
    int32_t* __restrict__ cnt, float* __restrict__ cd, int32_t* __restrict__ ci,
    float* __restrict__ fd) {
  constexpr int G = DT / 64;
  __shared__ float s_d[4][32][64];
  const int sl = blockIdx.x % S;
  const int nb = blockIdx.x / S;
  const int n = nb / nqb;
  const int w = wave_id(), lane = lane_id();
  const int qw = (nb - n * nqb) * 256 + 64 * w;
  if (qw >= P1) return;  // the whole wave
  const int q = qw + lane;
  int64_t l1 = len1[n], l2 = len2[n];
  l1 = l1 < 0 ? 0 : (l1 > P1 ? P1 : l1);
  l2 = l2 < 0 ? 0 : (l2 > P2 ? P2 : l2);
  const int L2 = (int)l2;
  const bool act = q < l1;  // l1 <= P1
  const size_t row = (size_t)n * P1 + min(q, P1 - 1);
  const size_t cs = row * S + sl;
  const int a = K + sl * slen, b = min(L2, a + slen);
  if (a >= b) {
    if (q < P1) cnt[cs] = 0;
    return;
  }
  const float* __restrict__ rp = p2 + (size_t)n * P2 * DT + 4 * (lane & 15);
  float qr[DT];
  {
    const float4* __restrict__ qp = reinterpret_cast<const float4*>(p1 + row * DT);
#pragma unroll
    for (int d = 0; d < DT / 4; ++d) {
      const float4 v = act ? qp[d] : make_float4(0.f, 0.f, 0.f, 0.f);
      qr[4 * d] = v.x;
      qr[4 * d + 1] = v.y;
      qr[4 * d + 2] = v.z;
      qr[4 * d + 3] = v.w;
    }
  }
  auto load_ref = [&](float4 (&rv)[G], int j) {
#pragma unroll
    for (int g = 0; g < G; ++g) rv[g] = *reinterpret_cast<const float4*>(rp + (size_t)j * DT + 64 * g);
  };
  constexpr auto dims = std::make_integer_sequence<int, DT>{};
  // the fill: references 0 .. K-1 (K < L2 here)
  float sd[KC];
#pragma unroll
  for (int t = 0; t < KC; ++t) {
    if (t < K) {
      float4 rv[G];
      load_ref(rv, t);
      sd[t] = hd_dist<NORM>(qr, rv, dims);
    } else {
      sd[t] = Lim<float>::inf();
    }
  }
  if (sl == 0 && act) {  // the merge's fill
#pragma unroll
    for (int t = 0; t < KC; ++t)
      if (t < K) fd[row * K + t] = sd[t];
  }
  float thr;
  int ms;
  first_max<float, KC>(sd, K, thr, ms);
  if (!act) thr = -Lim<float>::inf();  // no candidates
  int count = 0;
  float* __restrict__ cdp = cd + cs * HD_CAP;
  int32_t* __restrict__ cip = ci + cs * HD_CAP;

  // a ring of HD_J references in flight: buffer u holds reference
  // j = u (mod HD_J) and is reloaded with j + HD_J once its distance is taken
  float4 rb[HD_J][G];
#pragma unroll
  for (int u = 0; u < HD_J; ++u) load_ref(rb[u], min(a + u, b - 1));
  for (int base = a; base < b; base += 32) {
    uint32_t mask = 0;
    for (int u0 = 0; u0 < 32; u0 += HD_J) {
#pragma unroll
      for (int u = 0; u < HD_J; ++u) {
        float d = hd_dist<NORM>(qr, rb[u], dims);
        // the next reference for this buffer (clamped into the slice)
        load_ref(rb[u], min(base + u0 + HD_J + u, b - 1));
        d = base + u0 + u < b ? d : Lim<float>::inf();
        s_d[w][u0 + u][lane] = d;
        mask |= (d < thr ? 1u : 0u) << (u0 + u);
      }
    }
    // this lane's candidates in index order, against the current threshold
    while (mask != 0) {
      const int u = __builtin_ctz(mask);
      mask &= mask - 1;
      const float d = s_d[w][u][lane];
      if (d < thr) {
        if (count < HD_CAP) {
          cdp[count] = d;
          cip[count] = base + u;
        }
        ++count;
        mink_put<float, KC>(sd, ms, d);
        first_max<float, KC>(sd, K, thr, ms);
      }
    }
  }
  if (q < P1) cnt[cs] = act ? count : 0;
}

template <int DT, int NORM, int KC, bool SORT>
__global__ __launch_bounds__(256) void knn_hd_merge_kernel(
    const float* __restrict__ p1, const float* __restrict__ p2, const int64_t* __restrict__ len1,
    const int64_t* __restrict__ len2, int N, int P1, int P2, int K, int S, int slen, int pad_sentinel,
    const int32_t* __restrict__ cnt, const float* __restrict__ cd,
    const int32_t* __restrict__ ci, const float* __restrict__ fd, int64_t* __restrict__ idxs,
    float* __restrict__ dists) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)N * P1) return;
  const int n = (int)(t / P1), q = (int)(t - (int64_t)n * P1);
  int64_t l1 = len1[n], l2 = len2[n];
  l1 = l1 < 0 ? 0 : (l1 > P1 ? P1 : l1);
  l2 = l2 < 0 ? 0 : (l2 > P2 ? P2 : l2);
  const int L2 = (int)l2;
  const size_t row = (size_t)t;
  int64_t* __restrict__ io = idxs + row * K;
  float* __restrict__ dout = dists + row * K;
  if (q >= l1) {  // never written by the reference: its zeros
    for (int s = 0; s < K; ++s) {
      io[s] = 0;
      dout[s] = 0.f;
    }
    return;
  }
  // the query stays in memory (a register copy would be live through the
  // whole replay): distances here are the fill's and an overflowed slice's
  const float4* __restrict__ qp = reinterpret_cast<const float4*>(p1 + row * DT);
  const float* __restrict__ rp = p2 + (size_t)n * P2 * DT;
  auto dist = [&](int j) { return hd_dist_mem<NORM, DT>(qp, reinterpret_cast<const float4*>(rp + (size_t)j * DT)); };
  float sd[KC];
  int si[KC];
  const int fill = L2 < K ? L2 : K;
#pragma unroll
  for (int s = 0; s < KC; ++s) {
    if (s < fill) {
      // with more than K references the first slice stored them
      sd[s] = L2 > K ? fd[row * K + s] : dist(s);
      si[s] = s;
    } else {
      sd[s] = Lim<float>::inf();
      si[s] = -1;
    }
  }
  const int size = fill;
  if (L2 > K) {
    float thr;
    int ms;
    first_max<float, KC>(sd, K, thr, ms);
    auto replay = [&](float d, int j) {
      if (d < thr) {
        mink_put<float, KC>(sd, si, ms, d, j);
        first_max<float, KC>(sd, K, thr, ms);
      }
    };
    for (int sl = 0; sl < S; ++sl) {
      const int a = K + sl * slen, b = min(L2, a + slen);
      if (a >= b) break;
      const int c = cnt[row * S + sl];
      if (c <= HD_CAP) {
        // 16 candidates a step, loaded together (the list holds HD_CAP
        // entries, a multiple of 16, so a step never reads past it); the
        // step's mask against the threshold at its start is a superset of
        // its insertions, each re-checked against the current threshold
        const float4* __restrict__ cdp = reinterpret_cast<const float4*>(cd + (row * S + sl) * HD_CAP);
        const int4* __restrict__ cip = reinterpret_cast<const int4*>(ci + (row * S + sl) * HD_CAP);
        for (int k0 = 0; k0 < c; k0 += 16) {
          float dv[16];
          int iv[16];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float4 d4 = cdp[k0 / 4 + v];
            const int4 i4 = cip[k0 / 4 + v];
            dv[4 * v] = d4.x, dv[4 * v + 1] = d4.y, dv[4 * v + 2] = d4.z, dv[4 * v + 3] = d4.w;
            iv[4 * v] = i4.x, iv[4 * v + 1] = i4.y, iv[4 * v + 2] = i4.z, iv[4 * v + 3] = i4.w;
          }
          uint32_t m = 0;
#pragma unroll
          for (int e = 0; e < 16; ++e) m |= (k0 + e < c && dv[e] < thr ? 1u : 0u) << e;
          while (m != 0) {
            const int e = __builtin_ctz(m);
            m &= m - 1;
            float d = dv[0];
            int j = iv[0];
#pragma unroll
            for (int x = 1; x < 16; ++x) {
              d = x == e ? dv[x] : d;
              j = x == e ? iv[x] : j;
            }
            replay(d, j);
          }
        }
      } else {  // the slice's list overflowed: recompute it in order
        for (int j = a; j < b; ++j) replay(dist(j), j);
      }
    }
  }
  const int64_t pad_i = pad_sentinel ? -1 : 0;
  const float pad_d = pad_sentinel ? Lim<float>::inf() : 0.f;
  if constexpr (SORT) {
#pragma unroll
    for (int s = 0; s < KC; ++s) {
      if (s >= size) {
        sd[s] = Lim<float>::inf();
        si[s] = (int)pad_i;
      }
    }
    knn_sort_row<float, KC>(sd, si, K >= 32 ? 0xffffffffu : (1u << K) - 1u);
#pragma unroll
    for (int s = 0; s < KC; ++s) {
      if (s < K) {
        io[s] = (int64_t)si[s];
        dout[s] = s < size ? sd[s] : 0.f;
      }
    }
    return;
  }
#pragma unroll
  for (int s = 0; s < KC; ++s) {
    if (s < K) {
      io[s] = s < size ? (int64_t)si[s] : pad_i;
      dout[s] = s < size ? sd[s] : pad_d;
    }
  }
}

// S slices for the sliced high-D path, or 0 when it does not apply: float,
// D 64 or 128, 2 <= K <= 32, too few query workgroups to fill the GPU, and
// slices of at least 1024 references.
}  // namespace

int hd_slices(int dtype, int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K) {
  if (dtype != TPO_F32 || (D != 64 && D != 128) || K < 2 || K > 32) return 0;
  const int64_t wgs = N * ((P1 + 255) / 256);
  if (wgs <= 0 || wgs >= 256) return 0;
  int64_t S = 512 / wgs;
  S = S < 16 ? S : 16;
  const int64_t smax = (P2 - K) / 1024;
  S = S < smax ? S : smax;
  return S >= 2 ? (int)S : 0;
}

namespace {

template <int DT, int NORM, int KC>
void launch_hd_kc(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2, int N,
                  int P1, int P2, int K, int S, int pad, bool sort, int64_t* idxs, void* dists,
                  void* ws, hipStream_t s) {
  const int nqb = (P1 + 255) / 256;
  const int slen = (P2 - K + S - 1) / S;
  const HdLayout L = hd_layout((int64_t)N * P1, S, K);
  int32_t* cnt = (int32_t*)((char*)ws + L.cnt);
  float* cd = (float*)((char*)ws + L.dist);
  int32_t* ci = (int32_t*)((char*)ws + L.idx);
  float* fd = (float*)((char*)ws + L.fill);
  hipLaunchKernelGGL((knn_hd_slice_kernel<DT, NORM, KC>), dim3(N * nqb * S), dim3(256), 0, s,
                     (const float*)p1, (const float*)p2, l1, l2, P1, P2, K, nqb, S, slen, cnt, cd,
                     ci, fd);
  const unsigned mg = (unsigned)(((int64_t)N * P1 + 255) / 256);
  if (sort)
    hipLaunchKernelGGL((knn_hd_merge_kernel<DT, NORM, KC, true>), dim3(mg), dim3(256), 0, s,
                       (const float*)p1, (const float*)p2, l1, l2, N, P1, P2, K, S, slen, pad, cnt,
                       cd, ci, fd, idxs, (float*)dists);
  else
    hipLaunchKernelGGL((knn_hd_merge_kernel<DT, NORM, KC, false>), dim3(mg), dim3(256), 0, s,
                       (const float*)p1, (const float*)p2, l1, l2, N, P1, P2, K, S, slen, pad, cnt,
                       cd, ci, fd, idxs, (float*)dists);
}

template <int DT, int NORM>
void launch_hd_norm(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2, int N,
                    int P1, int P2, int K, int S, int pad, bool sort, int64_t* idxs, void* dists,
                    void* ws, hipStream_t s) {
  if (K <= 8) launch_hd_kc<DT, NORM, 8>(p1, p2, l1, l2, N, P1, P2, K, S, pad, sort, idxs, dists, ws, s);
  else if (K <= 16) launch_hd_kc<DT, NORM, 16>(p1, p2, l1, l2, N, P1, P2, K, S, pad, sort, idxs, dists, ws, s);
  else launch_hd_kc<DT, NORM, 32>(p1, p2, l1, l2, N, P1, P2, K, S, pad, sort, idxs, dists, ws, s);
}

}  // namespace

int64_t hd_workspace_bytes(int64_t rows, int64_t S, int64_t K) {
  return hd_layout(rows, S, K).total;
}

void launch_hd(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2, int N, int P1,
               int P2, int D, int K, int norm, int S, int pad, bool sort, int64_t* idxs,
               void* dists, void* ws, hipStream_t s) {
  if (D == 128) {
    if (norm == 1) launch_hd_norm<128, 1>(p1, p2, l1, l2, N, P1, P2, K, S, pad, sort, idxs, dists, ws, s);
    else launch_hd_norm<128, 2>(p1, p2, l1, l2, N, P1, P2, K, S, pad, sort, idxs, dists, ws, s);
  } else {
    if (norm == 1) launch_hd_norm<64, 1>(p1, p2, l1, l2, N, P1, P2, K, S, pad, sort, idxs, dists, ws, s);
    else launch_hd_norm<64, 2>(p1, p2, l1, l2, N, P1, P2, K, S, pad, sort, idxs, dists, ws, s);
  }
}


}  // namespace tpo
