// knn.hip -- K nearest neighbours (forward) for gfx950; the backward is in
// knn_bwd.hip.
//
// Forward (replaces KNearestNeighborKernelV0..V3, knn.cu:16-227).
//   One query per lane; the wave's 64 queries belong to one cloud, so the
//   reference cloud is walked in the same order by every lane and each
//   reference point is a wave-uniform scalar load (SGPRs, no LDS).
//   The output must be the reference's MinK slot layout (mink.cuh:77-121),
//   which depends on the whole insertion history, so every lane replays the
//   MinK process exactly: the first K references fill the slots in order; a
//   later reference replaces the FIRST slot holding the maximum when it is
//   strictly smaller.  To keep the wave from executing the O(K) slot update
//   whenever any one lane needs it, references are processed in chunks of 32:
//   the distances of a chunk are compared against the lane's current maximum
//   into a 32-bit candidate mask (the maximum only decreases, so the mask is
//   a superset of the real insertions); then each lane walks its own
//   candidates in index order, re-checking against the updated maximum.  The
//   wave pays for max-over-lanes(candidates per chunk), which after the first
//   few hundred references is 0-2 per chunk.
//   Version semantics (dispatch.cuh:106-147): all versions select the same
//   set except version 3 with K == 2 (RegisterMinK<2>, mink.cuh:212-265,
//   keeps the pair sorted); versions 0/1 pad missing slots with (-1, +inf),
//   versions 2/3 with (0, 0); rows >= lengths1 are (0, 0).
//   K > 32 (versions 0/1 only) keeps the slots in the output rows, like the
//   reference's global-memory MinK.
#include <utility>

#include "knn_common.hpp"

namespace tpo {
// knn_bf16.hip
int64_t knn_bf16_workspace(int64_t N, int64_t P1, int64_t P2, int64_t K);
bool knn_bf16_supported(int64_t D, int64_t K, int norm);
void launch_knn_bf16(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2, int N,
                     int P1, int P2, int D, int K, int64_t* idxs, void* dists, void* ws,
                     hipStream_t s);
// knn_grid.hip
bool knn_grid_applies(int dtype, int64_t D, int64_t K, int64_t P2);
int64_t knn_grid_workspace(int64_t N, int64_t P2);
void launch_knn_grid(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2,
                     int32_t* order, int N, int P1, int P2, int K, int norm, int pad,
                     bool sort, int64_t* idxs, void* dists, void* ws, hipStream_t s);
}  // namespace tpo

#pragma clang fp contract(off)

namespace tpo {
namespace {

// Per cloud, the valid queries (row < lengths1) in Morton order of a 16^3
// grid over their bounding box.  The order only decides which queries share
// a wave: neighbouring queries share their nearest references, so the MinK
// insertions of a wave's lanes coincide and the candidate loop below runs
// fewer iterations.  Results are bit-identical in any order.
constexpr int KNN_GRID = 16;
constexpr int KNN_CELLS = KNN_GRID * KNN_GRID * KNN_GRID;

template <typename T>
__global__ __launch_bounds__(1024) void knn_order_kernel(const T* __restrict__ p1,
                                                         const int64_t* __restrict__ len1, int P1,
                                                         int32_t* __restrict__ order) {
  __shared__ uint32_t cnt[KNN_CELLS];
  __shared__ float red[6][16];
  __shared__ uint32_t part[16];
  const int n = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int64_t l1 = len1[n];
  const int L1 = (int)(l1 < 0 ? 0 : (l1 > P1 ? P1 : l1));
  const T* __restrict__ P = p1 + (size_t)n * P1 * 3;
  int32_t* __restrict__ out = order + (size_t)n * P1;
  float lo[3] = {__builtin_inff(), __builtin_inff(), __builtin_inff()};
  float hi[3] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
  for (int k = tid; k < L1; k += 1024)
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const float v = (float)P[3 * k + c];
      lo[c] = fminf(lo[c], v);
      hi[c] = fmaxf(hi[c], v);
    }
#pragma unroll
  for (int c = 0; c < 3; ++c)
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      lo[c] = fminf(lo[c], __shfl_xor(lo[c], m, 64));
      hi[c] = fmaxf(hi[c], __shfl_xor(hi[c], m, 64));
    }
  if (lane == 0)
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      red[c][w] = lo[c];
      red[3 + c][w] = hi[c];
    }
  for (int c = tid; c < KNN_CELLS; c += 1024) cnt[c] = 0;
  __syncthreads();
  float glo[3], gs[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    float a = __builtin_inff(), z = -__builtin_inff();
    for (int v = 0; v < 16; ++v) {
      a = fminf(a, red[c][v]);
      z = fmaxf(z, red[3 + c][v]);
    }
    glo[c] = a;
    const float ext = z - a;
    gs[c] = (ext > 0.f && ext < __builtin_inff()) ? (float)KNN_GRID / ext : 0.f;
  }
  auto cell_of = [&](int k) -> uint32_t {
    uint32_t code = 0;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const float f = ((float)P[3 * k + c] - glo[c]) * gs[c];
      int i = (f == f) ? (int)f : 0;
      i = i < 0 ? 0 : (i > KNN_GRID - 1 ? KNN_GRID - 1 : i);
      uint32_t v = (uint32_t)i;
      v = (v | (v << 4)) & 0x0c3;
      v = (v | (v << 2)) & 0x249;
      code |= v << c;
    }
    return code;
  };
  for (int k = tid; k < L1; k += 1024) atomicAdd(&cnt[cell_of(k)], 1u);
  __syncthreads();
  {  // exclusive scan, 4 cells per thread
    uint32_t v[4], sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = cnt[tid * 4 + i];
      sum += v[i];
    }
    uint32_t incl = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t o = (uint32_t)__shfl_up((int)incl, d, 64);
      if (lane >= d) incl += o;
    }
    if (lane == 63) part[w] = incl;
    __syncthreads();
    uint32_t run = incl - sum;
    for (int v2 = 0; v2 < w; ++v2) run += part[v2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      cnt[tid * 4 + i] = run;
      run += v[i];
    }
  }
  __syncthreads();
  for (int k = tid; k < L1; k += 1024) out[atomicAdd(&cnt[cell_of(k)], 1u)] = k;
  for (int k = L1 + tid; k < P1; k += 1024) out[k] = k;  // rows past lengths1 keep their place
}

// mode bit 0: RegisterMinK<2> (version 3, K = 2); bit 1 (= SORT): rows
// sorted as knn_points(return_sorted=True) returns them (knn_sort_row).
template <typename T, int DT, int NORM, int KC, bool SORT>
__global__ __launch_bounds__(256) void knn_fwd_kernel(
    const T* __restrict__ p1, const T* __restrict__ p2, const int64_t* __restrict__ len1,
    const int64_t* __restrict__ len2, const int32_t* __restrict__ order, int P1, int P2, int D,
    int K, int nqb, int pad_sentinel, int mode, int64_t* __restrict__ idxs,
    T* __restrict__ dists) {
  const int sorted2 = mode & 1;
  // float D=3: reference points reach the lanes through a wave-private LDS
  // block (each lane stages one, every lane reads them back as broadcasts),
  // so the whole wave takes part in every chunk; lanes without a query run
  // along with a dummy one and an empty candidate threshold
  constexpr bool STAGED = DT == 3 && sizeof(T) == 4;
  __shared__ float4 s_ref[STAGED ? 4 : 1][64];
  const int n = blockIdx.x / nqb;
  const int i = (blockIdx.x - n * nqb) * 256 + threadIdx.x;  // position in processing order
  const bool in_range = i < P1;
  if (!STAGED && !in_range) return;
  const int q = in_range ? (order ? order[(size_t)n * P1 + i] : i) : 0;  // query row of this lane
  int64_t l1 = len1[n], l2 = len2[n];
  l1 = l1 < 0 ? 0 : (l1 > P1 ? P1 : l1);
  l2 = l2 < 0 ? 0 : (l2 > P2 ? P2 : l2);
  const int L2 = (int)l2;
  const size_t row = (size_t)n * P1 + q;
  int64_t* __restrict__ io = idxs + row * K;
  T* __restrict__ dout = dists + row * K;
  const bool act = in_range && q < l1;
  if (in_range && !act) {  // never written by the reference: its zeros
    for (int s = 0; s < K; ++s) {
      io[s] = 0;
      dout[s] = (T)0;
    }
  }
  if (!STAGED && !act) return;
  // rows past lengths1 sit at the end of the processing order: a wave with
  // no query left has nothing to stage for
  if (STAGED && __ballot(act) == 0) return;
  const int Dd = DT > 0 ? DT : D;
  const T* __restrict__ qp = p1 + row * Dd;
  const T* __restrict__ rp = p2 + (size_t)n * P2 * Dd;
  T qr[DT > 0 ? DT : 1];
  if constexpr (DT > 0) {
#pragma unroll
    for (int d = 0; d < DT; ++d) qr[d] = qp[d];
  }

  T sd[KC];
  int si[KC];
  int size = 0;
  if (sorted2) {
    // RegisterMinK<.., 2>::add, mink.cuh:221-248
    T d0 = Lim<T>::inf(), d1 = Lim<T>::inf();
    int i0 = -1, i1 = -1;
    for (int j = 0; j < L2; ++j) {
      const T d = knn_dist<T, DT, NORM>(qr, qp, rp + (size_t)j * Dd, D);
      if (j == 0) {
        d0 = d;
        i0 = 0;
      } else if (d < d0) {  // shift down, new pair head
        d1 = d0;
        i1 = i0;
        d0 = d;
        i0 = j;
      } else if (j == 1 || d < d1) {  // second slot (always taken for j == 1)
        d1 = d;
        i1 = j;
      }
    }
#pragma unroll
    for (int s = 0; s < KC; ++s) {
      sd[s] = s == 0 ? d0 : d1;
      si[s] = s == 0 ? i0 : i1;
    }
    size = L2 < 2 ? L2 : 2;
  } else {
    // fill phase: slot s <- reference s
    const int fill = L2 < K ? L2 : K;
#pragma unroll
    for (int s = 0; s < KC; ++s) {
      if (s < fill) {
        sd[s] = knn_dist<T, DT, NORM>(qr, qp, rp + (size_t)s * Dd, D);
        si[s] = s;
      } else {
        sd[s] = Lim<T>::inf();
        si[s] = -1;
      }
    }
    size = fill;
    if (L2 > K) {
      T thr;
      int ms;
      first_max<T, KC>(sd, K, thr, ms);
      if (!act) thr = -Lim<T>::inf();  // a lane without a query has no candidates
      // STAGED: references j0 .. j0 + 63 of a 64-reference stage sit in
      // s_ref[wave]; each lane's next one is loaded a stage ahead
      const int wv = threadIdx.x >> 6, ln = threadIdx.x & 63;
      float pf[3] = {0.f, 0.f, 0.f};
      auto prefetch = [&](int jb) {
        if constexpr (STAGED) {
          const T* __restrict__ r = rp + (size_t)min(jb + ln, L2 - 1) * 3;
          pf[0] = (float)r[0];
          pf[1] = (float)r[1];
          pf[2] = (float)r[2];
        }
      };
      prefetch(K);
      for (int j0 = K; j0 < L2; j0 += KNN_CHUNK) {
        const int cn = min(KNN_CHUNK, L2 - j0);
        const int ph = (j0 - K) & 63;  // position of the chunk in its stage
        if constexpr (STAGED) {
          if (ph == 0) {  // the wave's previous reads of s_ref[wv] precede this write
            s_ref[wv][ln] = make_float4(pf[0], pf[1], pf[2], 0.f);
            __builtin_amdgcn_wave_barrier();
            prefetch(j0 + 64);
          }
        }
        // distances of the chunk stay in registers (+inf past cn); bit 31-c
        // of mask flags reference j0+c as a candidate against the current
        // maximum
        T dch[KNN_CHUNK];
        if (STAGED && cn == KNN_CHUNK) {
#pragma unroll
          for (int c = 0; c < KNN_CHUNK; ++c) {
            const float4 r4 = s_ref[STAGED ? wv : 0][ph + c];
            const T rv[3] = {(T)r4.x, (T)r4.y, (T)r4.z};
            dch[c] = knn_dist<T, DT, NORM>(qr, qp, rv, D);
          }
        } else if (cn == KNN_CHUNK) {
#pragma unroll
          for (int c = 0; c < KNN_CHUNK; ++c) {
            const T* __restrict__ r = rp + (size_t)(j0 + c) * Dd;
            if constexpr (DT == 3) {
              const T rv[3] = {to_vgpr(r[0]), to_vgpr(r[1]), to_vgpr(r[2])};
              dch[c] = knn_dist<T, DT, NORM>(qr, qp, rv, D);
            } else {
              dch[c] = knn_dist<T, DT, NORM>(qr, qp, r, D);
            }
          }
        } else {
#pragma unroll
          for (int c = 0; c < KNN_CHUNK; ++c) {
            if (c < cn)
              dch[c] = knn_dist<T, DT, NORM>(qr, qp, rp + (size_t)(j0 + c) * Dd, D);
            else
              dch[c] = Lim<T>::inf();
          }
        }
        uint32_t mask = 0;
#pragma unroll
        for (int c = 0; c < KNN_CHUNK; c += 4)
          mask = push_lt4(mask, dch[c], dch[c + 1], dch[c + 2], dch[c + 3], thr);
        while (mask) {
          const int top = 31 - __builtin_clz(mask);  // earliest candidate first
          mask ^= 1u << top;
          const int c = KNN_CHUNK - 1 - top;
          const T d = select32(dch, c);
          if (d < thr) {
            mink_put<T, KC>(sd, si, ms, d, j0 + c);
            first_max<T, KC>(sd, K, thr, ms);
          }
        }
      }
    }
  }
  if (!act) return;
  const int64_t pad_i = pad_sentinel ? -1 : 0;
  const T pad_d = pad_sentinel ? Lim<T>::inf() : (T)0;
  if constexpr (SORT) {
    // the module's sort: slots past the reference count key as +inf, sort
    // last and read 0 afterwards (knn/__init__.py:111-131)
#pragma unroll
    for (int s = 0; s < KC; ++s) {
      if (s >= size) {
        sd[s] = Lim<T>::inf();
        si[s] = (int)pad_i;
      }
    }
    knn_sort_row<T, KC>(sd, si, K >= 32 ? 0xffffffffu : (1u << K) - 1u);
#pragma unroll
    for (int s = 0; s < KC; ++s) {
      if (s < K) {
        io[s] = (int64_t)si[s];
        dout[s] = s < size ? sd[s] : (T)0;
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

// ------------------------------------------ high-D float, references sliced
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

// K > 32: MinK held in the output row (the reference's V0/V1 layout).
template <typename T, int NORM>
__global__ __launch_bounds__(256) void knn_fwd_global_kernel(
    const T* __restrict__ p1, const T* __restrict__ p2, const int64_t* __restrict__ len1,
    const int64_t* __restrict__ len2, int P1, int P2, int D, int K, int nqb,
    int64_t* __restrict__ idxs, T* __restrict__ dists) {
  const int n = blockIdx.x / nqb;
  const int q = (blockIdx.x - n * nqb) * 256 + threadIdx.x;
  if (q >= P1) return;
  int64_t l1 = len1[n], l2 = len2[n];
  l1 = l1 < 0 ? 0 : (l1 > P1 ? P1 : l1);
  l2 = l2 < 0 ? 0 : (l2 > P2 ? P2 : l2);
  const size_t row = (size_t)n * P1 + q;
  int64_t* __restrict__ io = idxs + row * K;
  T* __restrict__ dout = dists + row * K;
  if (q >= l1) {
    for (int s = 0; s < K; ++s) {
      io[s] = 0;
      dout[s] = (T)0;
    }
    return;
  }
  for (int s = 0; s < K; ++s) {  // mink.cuh:83-86
    io[s] = -1;
    dout[s] = Lim<T>::inf();
  }
  const T* __restrict__ qp = p1 + row * D;
  const T* __restrict__ rp = p2 + (size_t)n * P2 * D;
  T thr = Lim<T>::inf();
  int ms = 0, size = 0;
  for (int j = 0; j < (int)l2; ++j) {
    const T d = knn_dist<T, 0, NORM>(nullptr, qp, rp + (size_t)j * D, D);
    if (size < K) {
      dout[size] = d;
      io[size] = j;
      ++size;
      if (size == K) {
        thr = dout[0];
        ms = 0;
        for (int s = 1; s < K; ++s)
          if (dout[s] > thr) {
            thr = dout[s];
            ms = s;
          }
      }
    } else if (d < thr) {
      dout[ms] = d;
      io[ms] = j;
      thr = dout[0];
      ms = 0;
      for (int s = 1; s < K; ++s)
        if (dout[s] > thr) {
          thr = dout[s];
          ms = s;
        }
    }
  }
}

template <typename T, int DT, int NORM, int KC>
void launch_fwd_kc(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2,
                   const int32_t* order, int N, int P1, int P2, int D, int K, int pad,
                   int sorted2, int64_t* idxs, void* dists, hipStream_t s) {
  const int nqb = (P1 + 255) / 256;
  if (sorted2 & 2)
    hipLaunchKernelGGL((knn_fwd_kernel<T, DT, NORM, KC, true>), dim3(N * nqb), dim3(256), 0, s,
                       (const T*)p1, (const T*)p2, l1, l2, order, P1, P2, D, K, nqb, pad, sorted2,
                       idxs, (T*)dists);
  else
    hipLaunchKernelGGL((knn_fwd_kernel<T, DT, NORM, KC, false>), dim3(N * nqb), dim3(256), 0, s,
                       (const T*)p1, (const T*)p2, l1, l2, order, P1, P2, D, K, nqb, pad, sorted2,
                       idxs, (T*)dists);
}

template <typename T, int DT, int NORM>
void launch_fwd_dt(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2,
                   const int32_t* order, int N, int P1, int P2, int D, int K, int pad,
                   int sorted2, int64_t* idxs, void* dists, hipStream_t s) {
  if (K <= 4) launch_fwd_kc<T, DT, NORM, 4>(p1, p2, l1, l2, order, N, P1, P2, D, K, pad, sorted2, idxs, dists, s);
  else if (K <= 8) launch_fwd_kc<T, DT, NORM, 8>(p1, p2, l1, l2, order, N, P1, P2, D, K, pad, sorted2, idxs, dists, s);
  else if (K <= 16) launch_fwd_kc<T, DT, NORM, 16>(p1, p2, l1, l2, order, N, P1, P2, D, K, pad, sorted2, idxs, dists, s);
  else launch_fwd_kc<T, DT, NORM, 32>(p1, p2, l1, l2, order, N, P1, P2, D, K, pad, sorted2, idxs, dists, s);
}

template <typename T, int NORM>
void launch_fwd_norm(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2,
                     int32_t* order, int N, int P1, int P2, int D, int K, int pad, int sorted2,
                     int64_t* idxs, void* dists, hipStream_t s) {
  if (K > 32) {
    const int nqb = (P1 + 255) / 256;
    hipLaunchKernelGGL((knn_fwd_global_kernel<T, NORM>), dim3(N * nqb), dim3(256), 0, s,
                       (const T*)p1, (const T*)p2, l1, l2, P1, P2, D, K, nqb, idxs, (T*)dists);
  } else if (D == 3) {
    if (order)
      hipLaunchKernelGGL(knn_order_kernel<T>, dim3(N), dim3(1024), 0, s, (const T*)p1, l1, P1,
                         order);
    launch_fwd_dt<T, 3, NORM>(p1, p2, l1, l2, order, N, P1, P2, D, K, pad, sorted2, idxs, dists, s);
  } else {
    if constexpr (sizeof(T) == 4) {  // common high-D widths: float query held in VGPRs
      if (D == 128) {
        launch_fwd_dt<T, 128, NORM>(p1, p2, l1, l2, nullptr, N, P1, P2, D, K, pad, sorted2, idxs, dists, s);
        return;
      }
      if (D == 64) {
        launch_fwd_dt<T, 64, NORM>(p1, p2, l1, l2, nullptr, N, P1, P2, D, K, pad, sorted2, idxs, dists, s);
        return;
      }
    }
    launch_fwd_dt<T, 0, NORM>(p1, p2, l1, l2, nullptr, N, P1, P2, D, K, pad, sorted2, idxs, dists, s);
  }
}

template <typename T>
void launch_fwd(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2,
                int32_t* order, int N, int P1, int P2, int D, int K, int norm, int pad,
                int sorted2, int64_t* idxs, void* dists, hipStream_t s) {
  if (norm == 1) launch_fwd_norm<T, 1>(p1, p2, l1, l2, order, N, P1, P2, D, K, pad, sorted2, idxs, dists, s);
  else launch_fwd_norm<T, 2>(p1, p2, l1, l2, order, N, P1, P2, D, K, pad, sorted2, idxs, dists, s);
}

// dispatch.cuh:114-147
bool check_version(int v, int64_t D, int64_t K) {
  if (v == 0) return true;
  if (v == 1) return D >= 1 && D <= 32;
  if (v == 2) return D >= 1 && D <= 8 && K >= 1 && K <= 32;
  if (v == 3) return D >= 1 && D <= 8 && K >= 1 && K <= 4;
  return false;
}
int choose_version(int64_t D, int64_t K) {
  for (int v = 3; v >= 1; --v)
    if (check_version(v, D, K)) return v;
  return 0;
}

}  // namespace
}  // namespace tpo

using namespace tpo;

extern "C" int64_t tpo_knn_workspace_size(int dtype, int64_t N, int64_t P1, int64_t P2,
                                          int64_t D, int64_t K, int norm) {
  if (N < 0 || P1 < 0 || P2 < 0 || D < 1 || K < 0) return -1;
  if (dtype == TPO_BF16) return knn_bf16_supported(D, K, norm) ? knn_bf16_workspace(N, P1, P2, K) : 0;
  int64_t order = ((N * P1 * 4 + 255) / 256) * 256;
  if (knn_grid_applies(dtype, D, K, P2)) order += knn_grid_workspace(N, P2);
  const int S = hd_slices(dtype, N, P1, P2, D, K);
  const int64_t hd = S > 0 ? hd_layout(N * P1, S, K).total : 0;
  return order > hd ? order : hd;
}

static int knn_fwd_impl(int dtype, const void* p1, const void* p2, const int64_t* lengths1,
                        const int64_t* lengths2, int64_t N, int64_t P1, int64_t P2, int64_t D,
                        int64_t K, int norm, int version, int64_t* idxs, void* dists,
                        int* version_out, void* workspace, int64_t workspace_bytes, void* stream,
                        bool sort_rows) {
  if (N < 0 || P1 < 0 || P2 < 0 || D < 1 || K < 0 || N >= (1 << 20) || P1 >= (1 << 30) ||
      P2 >= (1 << 30) || D >= (1 << 20) || K >= (1 << 20))
    return set_error(TPO_ERR_ARG, "tpo_knn_fwd: bad sizes");
  if (norm != 1 && norm != 2) return set_error(TPO_ERR_ARG, "Norm must be 1 or 2.");
  if (dtype == TPO_BF16) {  // matrix-core path (knn_bf16.hip); no reference version applies
    if (version_out) *version_out = -1;
    if (!knn_bf16_supported(D, K, norm))
      return set_error(TPO_ERR_DTYPE,
                       "tpo_knn_fwd: bfloat16 needs norm 2, D %% 8 == 0, 8 <= D <= 128, "
                       "1 <= K <= 32 (got norm %d, D %lld, K %lld)",
                       norm, (long long)D, (long long)K);
    if (N == 0 || P1 == 0) return TPO_OK;
    if (((uintptr_t)p1 | (uintptr_t)p2) & 15)
      return set_error(TPO_ERR_ARG, "tpo_knn_fwd: bfloat16 points must be 16-byte aligned");
    const int64_t need = knn_bf16_workspace(N, P1, P2, K);
    if (!workspace || workspace_bytes < need)
      return set_error(TPO_ERR_WORKSPACE, "tpo_knn_fwd: workspace of %lld bytes < %lld",
                       (long long)workspace_bytes, (long long)need);
    launch_knn_bf16(p1, p2, lengths1, lengths2, (int)N, (int)P1, (int)P2, (int)D, (int)K, idxs,
                    dists, workspace, (hipStream_t)stream);
    return check_launch("tpo_knn_fwd");
  }
  // knn.cu:332-338: invalid explicit versions are replaced by the automatic one
  int v = (version >= 0 && check_version(version, D, K)) ? version : choose_version(D, K);
  if (version_out) *version_out = v;
  if (N == 0 || P1 == 0 || K == 0) return TPO_OK;
  const int pad = v <= 1;
  const int sorted2 = (v == 3 && K == 2) | (sort_rows ? 2 : 0);  // the kernel's mode bits
  hipStream_t s = (hipStream_t)stream;
  {  // long reference clouds, few queries: references sliced over workgroups
    const int S = hd_slices(dtype, N, P1, P2, D, K);
    if (S > 0 && workspace && workspace_bytes >= hd_layout(N * P1, S, K).total && v <= 1) {
      launch_hd(p1, p2, lengths1, lengths2, (int)N, (int)P1, (int)P2, (int)D, (int)K, norm, S,
                pad, sort_rows, idxs, dists, workspace, s);
      return check_launch("tpo_knn_fwd");
    }
  }
  // the query ordering is an optimisation: without workspace, keep row order
  const int64_t order_bytes = ((N * P1 * 4 + 255) / 256) * 256;
  int32_t* order = (workspace && workspace_bytes >= N * P1 * 4) ? (int32_t*)workspace : nullptr;
  // float 3-D against long clouds: brute-force prefix, then a grid's candidates
  if (order && !(sorted2 & 1) && knn_grid_applies(dtype, D, K, P2) &&
      workspace_bytes >= order_bytes + knn_grid_workspace(N, P2)) {
    launch_knn_grid(p1, p2, lengths1, lengths2, order, (int)N, (int)P1, (int)P2, (int)K, norm, pad,
                    sort_rows, idxs, dists, (char*)workspace + order_bytes, s);
    return check_launch("tpo_knn_fwd");
  }
  switch (dtype) {
    case TPO_F32: launch_fwd<float>(p1, p2, lengths1, lengths2, order, (int)N, (int)P1, (int)P2, (int)D, (int)K, norm, pad, sorted2, idxs, dists, s); break;
    case TPO_F64: launch_fwd<double>(p1, p2, lengths1, lengths2, order, (int)N, (int)P1, (int)P2, (int)D, (int)K, norm, pad, sorted2, idxs, dists, s); break;
    case TPO_F16: launch_fwd<half_t>(p1, p2, lengths1, lengths2, order, (int)N, (int)P1, (int)P2, (int)D, (int)K, norm, pad, sorted2, idxs, dists, s); break;
    default: return set_error(TPO_ERR_DTYPE, "tpo_knn_fwd: unsupported dtype %d", dtype);
  }
  return check_launch("tpo_knn_fwd");
}

extern "C" int tpo_knn_fwd(int dtype, const void* p1, const void* p2, const int64_t* lengths1,
                           const int64_t* lengths2, int64_t N, int64_t P1, int64_t P2, int64_t D,
                           int64_t K, int norm, int version, int64_t* idxs, void* dists,
                           int* version_out, void* workspace, int64_t workspace_bytes,
                           void* stream) {
  return knn_fwd_impl(dtype, p1, p2, lengths1, lengths2, N, P1, P2, D, K, norm, version, idxs,
                      dists, version_out, workspace, workspace_bytes, stream, false);
}

extern "C" int tpo_knn_fwd_sorted(int dtype, const void* p1, const void* p2,
                                  const int64_t* lengths1, const int64_t* lengths2, int64_t N,
                                  int64_t P1, int64_t P2, int64_t D, int64_t K, int norm,
                                  int version, int64_t* idxs, void* dists, int* version_out,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
  if (dtype != TPO_F32 && dtype != TPO_F64 && dtype != TPO_F16)
    return set_error(TPO_ERR_DTYPE, "tpo_knn_fwd_sorted: unsupported dtype %d", dtype);
  if (K < 2 || K > 32)
    return set_error(TPO_ERR_ARG, "tpo_knn_fwd_sorted: needs 2 <= K <= 32 (got %lld)",
                     (long long)K);
  return knn_fwd_impl(dtype, p1, p2, lengths1, lengths2, N, P1, P2, D, K, norm, version, idxs,
                      dists, version_out, workspace, workspace_bytes, stream, true);
}

