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
// knn_hd.hip
int hd_slices(int dtype, int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K);
int64_t hd_workspace_bytes(int64_t rows, int64_t S, int64_t K);
void launch_hd(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2, int N, int P1,
               int P2, int D, int K, int norm, int S, int pad, bool sort, int64_t* idxs,
               void* dists, void* ws, hipStream_t s);
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
  const int64_t hd = S > 0 ? hd_workspace_bytes(N * P1, S, K) : 0;
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
    if (S > 0 && workspace && workspace_bytes >= hd_workspace_bytes(N * P1, S, K) && v <= 1) {
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

