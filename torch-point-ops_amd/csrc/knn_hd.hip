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
// slices, and a workgroup per (cloud, 256 queries, slice) keeps, over its
// slice only, the K smallest distances of the K fill references (0 .. K-1)
// and of the slice so far.  Those are K values of the real process's prefix,
// so their largest is at least the prefix's K-th smallest value, which the
// real threshold never exceeds (a NaN fill slot only removes a slot from the
// real process): every reference the real process inserts passes the local
// threshold, and the local candidates (distance, index) of a slice are a
// superset of the real insertions.
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
// reference is lane (d % 64) / 4 of the row, VGPR (d / 64, d % 4).  The
// differences are taken two at a time: a DPP subtraction whose destination
// the previous VALU op wrote needs two wait states (its old-value operand),
// and two live differences keep consecutive subtractions in different VGPRs.
template <int NORM, int DT, int D0>
__device__ __forceinline__ void hd_pair(float& acc, const float (&qr)[DT], const float4 (&rv)[DT / 64]) {
  constexpr int D1 = D0 + 1;
  const float x0 = qr[D0] - row_bcast<(D0 % 64) / 4>(f4_at<D0 % 4>(rv[D0 / 64]));
  const float x1 = qr[D1] - row_bcast<(D1 % 64) / 4>(f4_at<D1 % 4>(rv[D1 / 64]));
  acc = NORM == 2 ? knn_acc2(acc, x0, D0 == 0) : knn_acc1(acc, x0, D0 == 0);
  acc = NORM == 2 ? knn_acc2(acc, x1, false) : knn_acc1(acc, x1, false);
}
template <int NORM, int DT, int... P>
__device__ __forceinline__ float hd_dist(const float (&qr)[DT], const float4 (&rv)[DT / 64],
                                         std::integer_sequence<int, P...>) {
  float acc = 0.f;
  (hd_pair<NORM, DT, 2 * P>(acc, qr, rv), ...);
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
  constexpr auto dims = std::make_integer_sequence<int, DT / 2>{};
  // the fill: references 0 .. K-1 (K < L2 here)
  // the local threshold: the K smallest distances of the fill and of the
  // slice so far (NaN as +inf), sorted ascending in srt[KC - K .. KC - 1]
  // behind KC - K entries of -inf, so that srt[KC - 1] is the threshold.
  // Keeping d (below the threshold) drops the largest: entry s becomes the
  // median of entries s - 1, s and d, one v_med3 each.
  float srt[KC];
#pragma unroll
  for (int t = 0; t < KC; ++t) srt[t] = t < KC - K ? -Lim<float>::inf() : Lim<float>::inf();
  auto keep = [&](float d) {
#pragma unroll
    for (int t = KC - 1; t > 0; --t) srt[t] = __builtin_amdgcn_fmed3f(srt[t - 1], srt[t], d);
    srt[0] = fminf(srt[0], d);
  };
#pragma unroll
  for (int t = 0; t < KC; ++t) {
    if (t < K) {
      float4 rv[G];
      load_ref(rv, t);
      const float d = hd_dist<NORM>(qr, rv, dims);
      if (sl == 0 && act) fd[row * K + t] = d;  // the merge's fill
      keep(d == d ? d : Lim<float>::inf());
    }
  }
  float thr = act ? srt[KC - 1] : -Lim<float>::inf();  // an idle lane has no candidates
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
    // the last walk's candidate stores count on vmcnt too: settle them here,
    // so that within the chunk each reference waits only for its own loads
    // (issued HD_J - 1 distances earlier) and not for the newest ones
    __builtin_amdgcn_s_waitcnt(0);
    for (int u0 = 0; u0 < 32; u0 += HD_J) {
#pragma unroll
      for (int u = 0; u < HD_J; ++u) {
        // an ordering point: the loads issued so far stay above it and this
        // reference's distance below, so each buffer is reloaded right after
        // its distance instead of all HD_J at the end of the step
#pragma unroll
        for (int g = 0; g < G; ++g)
          asm volatile("" : "+v"(rb[u][g].x), "+v"(rb[u][g].y), "+v"(rb[u][g].z), "+v"(rb[u][g].w) :: "memory");
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
        keep(d);
        thr = srt[KC - 1];
      }
    }
  }
  if (q < P1) cnt[cs] = act ? count : 0;
}

// The merge runs one wave per query row.  The replay's K slots live one per
// lane (lanes 0 .. K-1) as a list ordered by (value, slot descending), NaN
// values first: the last lane then holds the slot that first_max picks (the
// first slot holding the largest value; a NaN never becomes the maximum
// unless it sits in slot 0, and then the threshold is NaN and nothing is
// ever inserted).  Inserting (d, j) below the threshold puts it into the
// last element's slot: the lanes whose key exceeds the new one shift up one
// lane (DPP wave_shr) and the new entry lands in the gap.  Candidates come
// 64 at a time, one per lane; a ballot against the threshold finds the next
// insertion in index order, and is taken again after each one.

// order key of a distance: the compare-equal floats share one (-0 as +0),
// NaN below every number
__device__ __forceinline__ uint32_t hd_ord(float v) {
  const uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);
  return v != v ? 0u : ((u & 0x80000000u) ? ~u : (u | 0x80000000u));
}
__device__ __forceinline__ int hd_shr1(int x) {  // lane i takes lane i-1 (lane 0: 0)
  return __builtin_amdgcn_mov_dpp(x, 0x138, 0xF, 0xF, true);
}
__device__ __forceinline__ int hd_lane(int x, int l) { return __builtin_amdgcn_readlane(x, l); }
__device__ __forceinline__ float hd_lane(float x, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}

template <int DT, int NORM, int KC, bool SORT>
__global__ __launch_bounds__(256) void knn_hd_merge_kernel(
    const float* __restrict__ p1, const float* __restrict__ p2, const int64_t* __restrict__ len1,
    const int64_t* __restrict__ len2, int N, int P1, int P2, int K, int S, int slen, int pad_sentinel,
    const int32_t* __restrict__ cnt, const float* __restrict__ cd,
    const int32_t* __restrict__ ci, const float* __restrict__ fd, int64_t* __restrict__ idxs,
    float* __restrict__ dists) {
  const int64_t row = (int64_t)blockIdx.x * 4 + wave_id();
  if (row >= (int64_t)N * P1) return;  // the whole wave
  const int lane = lane_id();
  const int n = (int)(row / P1), q = (int)(row - (int64_t)n * P1);
  int64_t l1 = len1[n], l2 = len2[n];
  l1 = l1 < 0 ? 0 : (l1 > P1 ? P1 : l1);
  l2 = l2 < 0 ? 0 : (l2 > P2 ? P2 : l2);
  const int L2 = (int)l2;
  int64_t* __restrict__ io = idxs + row * K;
  float* __restrict__ dout = dists + row * K;
  if (q >= l1) {  // never written by the reference: its zeros
    if (lane < K) {
      io[lane] = 0;
      dout[lane] = 0.f;
    }
    return;
  }
  const float4* __restrict__ qp = reinterpret_cast<const float4*>(p1 + row * DT);
  const float* __restrict__ rp = p2 + (size_t)n * P2 * DT;
  auto dist = [&](int j) { return hd_dist_mem<NORM, DT>(qp, reinterpret_cast<const float4*>(rp + (size_t)j * DT)); };
  // lane s < K: slot s of the fill (with more than K references the first
  // slice stored its distances)
  const int fill = L2 < K ? L2 : K;
  float v = Lim<float>::inf();
  int ix = -1;
  if (lane < fill) {
    v = L2 > K ? fd[row * K + lane] : dist(lane);
    ix = lane;
  }
  if (L2 > K && hd_lane(v, 0) == hd_lane(v, 0)) {
    // the fill as the ordered list: lane s moves to its rank.  An entry is
    // (value, slot << 26 | index) (references fewer than 2^26).
    const uint64_t key = ((uint64_t)hd_ord(v) << 32) | (uint32_t)(63 - lane);
    int rank = 0;
#pragma unroll
    for (int t = 0; t < KC; ++t) {
      if (t < K) {
        const uint64_t kt = ((uint64_t)(uint32_t)hd_lane((int)(key >> 32), t) << 32) |
                            (uint32_t)hd_lane((int)(uint32_t)key, t);
        rank += kt < key ? 1 : 0;
      }
    }
    const int to = 4 * (lane < K ? rank : lane);
    v = __int_as_float(__builtin_amdgcn_ds_permute(to, __float_as_int(v)));
    int pk = __builtin_amdgcn_ds_permute(to, (lane << 26) | ix);
    float thr = hd_lane(v, K - 1);
    // (d, j) takes the last entry's slot; the entries after it in the order
    // (a larger value, or an equal one in a lower slot) move up one lane
    auto insert = [&](float d, int j) {
      const int sr = hd_lane(pk, K - 1) & ~0x3ffffff;
      const float vp = __int_as_float(hd_shr1(__float_as_int(v)));
      const int pp = hd_shr1(pk);
      // bitwise, not short-circuit: no branches in the wave-wide step
      const bool in = lane < K;
      const bool gt = in & ((v > d) | ((v == d) & (pk < sr)));
      const bool gtp = in & (lane > 0) & ((vp > d) | ((vp == d) & (pp < sr)));
      v = gtp ? vp : (gt ? d : v);
      pk = gtp ? pp : (gt ? (sr | j) : pk);
      thr = hd_lane(v, K - 1);
    };
    // one candidate per lane, in index order across the lanes
    auto batch = [&](float di, int ji, bool ok) {
      uint64_t m = __ballot(ok && di < thr);
      while (m != 0) {
        const int e = __builtin_ctzll(m);
        insert(hd_lane(di, e), hd_lane(ji, e));
        m &= __ballot(ok && di < thr) & ~((2ull << e) - 1ull);
      }
    };
    for (int sl = 0; sl < S; ++sl) {
      const int a = K + sl * slen, b = min(L2, a + slen);
      if (a >= b) break;
      const int c = cnt[row * S + sl];
      if (c <= HD_CAP) {
        const float* __restrict__ cdp = cd + (row * S + sl) * HD_CAP;
        const int32_t* __restrict__ cip = ci + (row * S + sl) * HD_CAP;
        for (int k0 = 0; k0 < c; k0 += 64) {
          const int k = min(k0 + lane, c - 1);  // lanes past the list repeat its last entry
          batch(cdp[k], cip[k], k0 + lane < c);
        }
      } else {  // the slice's list overflowed: recompute it in order
        for (int j0 = a; j0 < b; j0 += 64) {
          const int j = min(j0 + lane, b - 1);
          batch(dist(j), j, j0 + lane < b);
        }
      }
    }
    // back to slot order: lane s takes slot s
    const int back = 4 * (lane < K ? (pk >> 26) : lane);
    v = __int_as_float(__builtin_amdgcn_ds_permute(back, __float_as_int(v)));
    ix = __builtin_amdgcn_ds_permute(back, pk) & 0x3ffffff;
  }
  const int size = fill;
  const int64_t pad_i = pad_sentinel ? -1 : 0;
  const float pad_d = pad_sentinel ? Lim<float>::inf() : 0.f;
  if constexpr (SORT) {
    // knn_sort_row's network with position p in lane p: an exchange of
    // positions (a, a + stride) runs in both lanes, which agree on it
    float d = lane < size ? v : Lim<float>::inf();
    int x = lane < size ? ix : (int)pad_i;
    int va = lane < K ? 1 : 0;
    auto cas = [&](int stride, bool up) {
      const float pd = __shfl_xor(d, stride);
      const int px = __shfl_xor(x, stride), pv = __shfl_xor(va, stride);
      const bool lo = (lane & stride) == 0;
      const float da = lo ? d : pd, db = lo ? pd : d;
      const bool vA = (lo ? va : pv) != 0, vB = (lo ? pv : va) != 0;
      const bool lt = !knn_isnan(da) && (knn_isnan(db) || da < db);
      const bool sw = ((lt && vA) || !vB) == up;
      if ((lane | stride) < KC && sw) {
        d = pd;
        x = px;
        va = pv;
      }
    };
#pragma unroll
    for (int sz = 2; sz < 32; sz *= 2)
#pragma unroll
      for (int stride = sz / 2; stride > 0; stride /= 2) cas(stride, (lane & sz) != 0);
#pragma unroll
    for (int stride = 16; stride > 0; stride /= 2) cas(stride, false);
    if (lane < K) {
      io[lane] = (int64_t)x;
      dout[lane] = lane < size ? d : 0.f;
    }
    return;
  }
  if (lane < K) {
    io[lane] = lane < size ? (int64_t)ix : pad_i;
    dout[lane] = lane < size ? v : pad_d;
  }
}

// S slices for the sliced high-D path, or 0 when it does not apply: float,
// D 64 or 128, 2 <= K <= 32, at most 2^26 references, too few query
// workgroups to fill the GPU, and slices of at least 1024 references.
}  // namespace

int hd_slices(int dtype, int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K) {
  if (dtype != TPO_F32 || (D != 64 && D != 128) || K < 2 || K > 32 || P2 > (1 << 26)) return 0;
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
  const unsigned mg = (unsigned)(((int64_t)N * P1 + 3) / 4);  // a wave per row
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
