// fps.hip -- furthest point sampling for gfx950.
//
// Replaces furthest_point_sampling_kernel (fps.cu:111-214).  Reference
// semantics reproduced exactly:
//   * idx[0] = 0; a point k takes part only if |p_k|^2 > 1e-3 (in the dtype,
//     fps.cu:142-143); its running minimum temp_k starts at 1e10 (1e4 for
//     fp16, fps.cu:291-292) and becomes min(d, temp_k) with
//     d = |p_k - p_old|^2 in the reference's arithmetic;
//   * the next sample is the point with the largest temp; ties go to the
//     lowest "rank", the closed form of the reference's reduction: its
//     thread tid = k mod BS scans k in increasing order keeping the first
//     strict maximum, and its shared-memory tree (fps.cu:155-209) keeps the
//     left operand on ties, which orders threads by bit-reversed tid.  So
//       rank(k) = bitrev_log2(BS)(k mod BS) * ceil(N/BS) + k / BS,
//       BS = min(512, 2^floor(log2 N)) (fps.cu:56-60);
//   * no participating point at all -> the sample is index 0.
//
// Design (one 1024-thread workgroup per cloud; no inter-workgroup sync):
//   1. The workgroup sorts its cloud into a workspace by Hilbert cell of a
//      16^3 grid (counting sort in LDS) and cuts the sorted order into
//      buckets of S = 64 points (S grows for N > 65536 so there are <= 1024).
//   2. Each lane owns one bucket: its bounding box and the bucket's best
//      (largest temp, lowest rank) candidate, in registers.
//   3. Per sample, a lane marks its bucket "touched" unless the squared
//      distance from the new point to the bucket's box provably exceeds the
//      bucket's largest temp (then min(d, temp) == temp for every point in
//      it; the test keeps a relative margin far above the rounding error of
//      d).  Each wave updates its touched buckets (64 lanes = 64 points),
//      re-reduces their best candidates, reduces over its 64 buckets, and
//      one barrier later every wave reduces the 16 wave results.
//   Work per sample drops from N points to the few buckets near the new
//   sample, while the result is bit-identical to the full sweep.  The first
//   sample (index 0) touches every point; its update is made in the set-up
//   pass that initialises the running minima, with the same arithmetic.
#include "tpo_common.hpp"

#pragma clang fp contract(off)

namespace tpo {
namespace {

constexpr int FPS_THREADS = 1024;
constexpr int FPS_WAVES = FPS_THREADS / 64;
constexpr int FPS_GRID = 16;  // cell grid per axis (4096 cells)
constexpr int FPS_CELLS = FPS_GRID * FPS_GRID * FPS_GRID;

// candidate/value type: float holds every binary16 and binary32 value exactly
template <typename T> struct FpsV { typedef float type; };
template <> struct FpsV<double> { typedef double type; };

template <typename T> struct FpsConst;
template <> struct FpsConst<float> {
  __device__ static float thr() { return 1e-3f; }
  __device__ static float init() { return 1e10f; }
  __device__ static float margin() { return 1e-5f; }
  __device__ static float tiny() { return 1e-30f; }
};
template <> struct FpsConst<double> {
  __device__ static double thr() { return 1e-3; }
  __device__ static double init() { return 1e10; }
  __device__ static double margin() { return 1e-12; }
  __device__ static double tiny() { return 1e-290; }
};
template <> struct FpsConst<half_t> {
  __device__ static half_t thr() { return (half_t)1e-3f; }
  __device__ static half_t init() { return (half_t)1e4f; }
  __device__ static float margin() { return 1e-2f; }
  __device__ static float tiny() { return 1e-3f; }
};

// One sorted point: coordinates and key = ~rank for a point that takes part,
// 0 for one that does not (its running minimum is then held at 0),
// loaded as a single 16-byte access for float.
template <typename T> struct FpsRec {
  T x, y, z;
  uint32_t key;
};

struct FpsLayout {
  int64_t np;      // padded points per cloud = nb * s
  int64_t stride;  // bytes per cloud
  int64_t off_r, off_t;
};

template <typename T>
__host__ __device__ inline FpsLayout fps_layout(int64_t n) {
  const int64_t s = 64 * ((n + 64 * FPS_THREADS - 1) / (64 * FPS_THREADS));
  const int64_t nb = (n + s - 1) / s;
  FpsLayout L;
  L.np = nb * s;
  auto al = [](int64_t v) { return (v + 255) / 256 * 256; };
  int64_t o = 0;
  L.off_r = o; o += al(L.np * (int64_t)sizeof(FpsRec<T>));
  L.off_t = o; o += al(L.np * (int64_t)sizeof(T));
  L.stride = o;
  return L;
}


// ------------------------------------------------------------ candidates
// A candidate is (running-min value, rank); the better one has the larger
// value, then the lower rank.  For float/half values (all >= +0) it is packed
// into one 64-bit key, (value bits << 32) | (0xffffffff - rank), so "better"
// is an unsigned compare and 0 means "no candidate"; wave reductions then run
// on DPP lane swizzles.  double values keep a (value, rank) pair.
struct CandF {
  uint64_t k;
};
struct CandD {
  double v;
  uint32_t r;
};
template <typename T> struct FpsCand { typedef CandF type; };
template <> struct FpsCand<double> { typedef CandD type; };

// key = ~rank, or 0 for "no candidate" (whose value is then +0)
__device__ __forceinline__ CandF cand_make(float v, uint32_t key, CandF*) {
  return {((uint64_t)__float_as_uint(v) << 32) | (uint64_t)key};
}
__device__ __forceinline__ CandD cand_make(double v, uint32_t key, CandD*) {
  return key ? CandD{v, ~key} : CandD{-1.0, 0xffffffffu};
}
__device__ __forceinline__ CandF cand_none(CandF*) { return {0}; }
__device__ __forceinline__ CandD cand_none(CandD*) { return {-1.0, 0xffffffffu}; }
__device__ __forceinline__ bool cand_gt(CandF a, CandF b) { return a.k > b.k; }
__device__ __forceinline__ bool cand_gt(CandD a, CandD b) {
  return a.v > b.v || (a.v == b.v && a.r < b.r);
}
__device__ __forceinline__ bool cand_eq(CandF a, CandF b) { return a.k == b.k; }
__device__ __forceinline__ bool cand_eq(CandD a, CandD b) { return a.v == b.v && a.r == b.r; }
__device__ __forceinline__ bool cand_valid(CandF a) { return a.k != 0; }
__device__ __forceinline__ bool cand_valid(CandD a) { return a.v >= 0.0; }
__device__ __forceinline__ float cand_val(CandF a) { return __uint_as_float((uint32_t)(a.k >> 32)); }
__device__ __forceinline__ double cand_val(CandD a) { return a.v; }
__device__ __forceinline__ uint32_t cand_rank(CandF a) { return 0xffffffffu - (uint32_t)a.k; }
__device__ __forceinline__ uint32_t cand_rank(CandD a) { return a.r; }
// the record key (~rank, 0 for none) of a candidate
__device__ __forceinline__ uint32_t cand_keyword(CandF a) { return (uint32_t)a.k; }
__device__ __forceinline__ uint32_t cand_keyword(CandD a) { return ~a.r; }

template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint32_t dpp_umax(uint32_t v) {
  // folds into one v_max_u32_dpp; lanes of masked-off rows keep v
  const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWMASK, 0xf, false);
  return o > v ? o : v;
}
// max over the 64 lanes (all active), in every lane
__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
  v = dpp_umax<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
  v = dpp_umax<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
  v = dpp_umax<0x141, 0xf>(v);  // row_half_mirror
  v = dpp_umax<0x140, 0xf>(v);  // row_mirror: each lane holds its row's max
  v = dpp_umax<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
  v = dpp_umax<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
// first lane whose candidate equals c (c is wave-uniform and held by a lane)
template <typename C>
__device__ __forceinline__ int lane_of(C mine, C c) {
  const uint64_t hit = __ballot(cand_eq(mine, c));
  return hit ? __builtin_ctzll(hit) : 0;
}

// Best candidate of the whole wave (double values: (value, rank) pairs).
__device__ __forceinline__ CandD wave_best(CandD c) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const CandD o = {__shfl_xor(c.v, m, 64), (uint32_t)__shfl_xor((int)c.r, m, 64)};
    if (cand_gt(o, c)) c = o;
  }
  return c;
}
// Best candidate of the wave and the (first) lane holding it.  The rank
// pass only runs when several lanes share the largest value.
__device__ __forceinline__ CandF wave_best_at(CandF c, int& wl) {
  const uint32_t hi = (uint32_t)(c.k >> 32);
  const uint32_t mh = wave_umax(hi);
  const uint64_t eq = __ballot(hi == mh);
  if (__builtin_popcountll(eq) == 1) {
    wl = __builtin_ctzll(eq);
    return {((uint64_t)mh << 32) | (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)c.k, wl)};
  }
  const uint32_t ml = wave_umax(hi == mh ? (uint32_t)c.k : 0u);
  const CandF b = {((uint64_t)mh << 32) | ml};
  wl = lane_of(c, b);
  return b;
}
__device__ __forceinline__ CandD wave_best_at(CandD c, int& wl) {
  const CandD b = wave_best(c);
  wl = lane_of(c, b);
  return b;
}
__device__ __forceinline__ CandD row0_best(CandD c) {
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) {
    const CandD o = {__shfl_xor(c.v, m, 64), (uint32_t)__shfl_xor((int)c.r, m, 64)};
    if (cand_gt(o, c)) c = o;
  }
  return {__shfl(c.v, 0, 64), (uint32_t)__shfl((int)c.r, 0, 64)};
}

__device__ __forceinline__ float vmax(float a, float b) { return fmaxf(a, b); }
__device__ __forceinline__ double vmax(double a, double b) { return fmax(a, b); }
__device__ __forceinline__ float vfma(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double vfma(double a, double b, double c) { return __builtin_fma(a, b, c); }

__device__ __forceinline__ float bcast(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ double bcast(double v, int lane) { return __shfl(v, lane, 64); }
__device__ __forceinline__ half_t bcast(half_t v, int lane) {
  return (half_t)bcast((float)v, lane);  // exact round trip
}


template <typename T>
__global__ __launch_bounds__(FPS_THREADS) void fps_kernel(const T* __restrict__ pts, int N, int m,
                                                          int bs, int bs_bits, int per,
                                                          char* __restrict__ ws,
                                                          int64_t* __restrict__ idx_out) {
  typedef typename FpsV<T>::type V;
  __shared__ uint32_t s_cnt[FPS_CELLS];
  __shared__ uint32_t s_part[FPS_THREADS / 64];
  __shared__ V s_red[6][FPS_WAVES];
  struct WaveBest {
    typename FpsCand<T>::type c;
    T x, y, z;
  };
  __shared__ WaveBest s_wb[2][FPS_WAVES];
  __shared__ unsigned long long s_gkey[3];

  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
  const FpsLayout L = fps_layout<T>(N);
  const int s_sz = (int)(64 * ((N + 64 * FPS_THREADS - 1) / (64 * FPS_THREADS)));
  const int nb = (N + s_sz - 1) / s_sz;
  char* base = ws + (size_t)b * L.stride;
  FpsRec<T>* __restrict__ recs = (FpsRec<T>*)(base + L.off_r);
  T* __restrict__ ts = (T*)(base + L.off_t);
  const T* __restrict__ P = pts + (size_t)b * N * 3;
  int64_t* __restrict__ out = idx_out + (size_t)b * m;

  // ---- 1. bounding box of the cloud (for the cell grid only) ----
  float lo[3] = {__builtin_inff(), __builtin_inff(), __builtin_inff()};
  float hi[3] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
  for (int k = tid; k < N; k += FPS_THREADS) {
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
    for (int mm = 32; mm >= 1; mm >>= 1) {
      lo[c] = fminf(lo[c], __shfl_xor(lo[c], mm, 64));
      hi[c] = fmaxf(hi[c], __shfl_xor(hi[c], mm, 64));
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      s_red[c][w] = (V)lo[c];
      s_red[3 + c][w] = (V)hi[c];
    }
  }
  for (int c = tid; c < FPS_CELLS; c += FPS_THREADS) s_cnt[c] = 0;
  if (tid < 3) s_gkey[tid] = 0;
  __syncthreads();
  float glo[3], gscale[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    float a = __builtin_inff(), z = -__builtin_inff();
    for (int v = 0; v < FPS_WAVES; ++v) {
      a = fminf(a, (float)s_red[c][v]);
      z = fmaxf(z, (float)s_red[3 + c][v]);
    }
    const float ext = z - a;
    glo[c] = a;
    gscale[c] = (ext > 0.f && ext < __builtin_inff()) ? (float)FPS_GRID / ext : 0.f;
  }

  // ---- 2. counting sort by the cells' Hilbert order ----
  auto cell_of = [&](int k) -> uint32_t {
    uint32_t cc[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      float f = ((float)P[3 * k + c] - glo[c]) * gscale[c];
      int i = (f == f) ? (int)f : 0;
      i = i < 0 ? 0 : (i > FPS_GRID - 1 ? FPS_GRID - 1 : i);
      cc[c] = (uint32_t)i;
    }
    return hilbert3_16(cc[0], cc[1], cc[2]);
  };
  for (int k = tid; k < N; k += FPS_THREADS) atomicAdd(&s_cnt[cell_of(k)], 1u);
  __syncthreads();
  {  // exclusive scan of 4096 counters: 4 per thread
    constexpr int PER = FPS_CELLS / FPS_THREADS;
    uint32_t v[PER], sum = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      v[i] = s_cnt[tid * PER + i];
      sum += v[i];
    }
    uint32_t incl = sum;  // wave inclusive scan
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t o = (uint32_t)__shfl_up((int)incl, d, 64);
      if (lane >= d) incl += o;
    }
    if (lane == 63) s_part[w] = incl;
    __syncthreads();
    uint32_t woff = 0;
    for (int v2 = 0; v2 < w; ++v2) woff += s_part[v2];
    uint32_t run = woff + incl - sum;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      s_cnt[tid * PER + i] = run;
      run += v[i];
    }
  }
  __syncthreads();
  const T thr = FpsConst<T>::thr();
  const T init = FpsConst<T>::init();
  for (int k = tid; k < N; k += FPS_THREADS) {
    const uint32_t pos = atomicAdd(&s_cnt[cell_of(k)], 1u);
    const T x = P[3 * k], y = P[3 * k + 1], z = P[3 * k + 2];
    const bool valid = sq3(x, y, z) > thr;  // fps.cu:142-143
    const uint32_t t = (uint32_t)(k & (bs - 1));
    const uint32_t rev = bs_bits ? (__builtin_bitreverse32(t) >> (32 - bs_bits)) : 0u;
    const uint32_t rank = rev * (uint32_t)per + (uint32_t)(k / bs);
    recs[pos] = FpsRec<T>{x, y, z, valid ? ~rank : 0u};
  }
  for (int64_t k = N + tid; k < L.np; k += FPS_THREADS) recs[k] = FpsRec<T>{(T)0, (T)0, (T)0, 0u};
  __syncthreads();
  // running minima in sorted order (coalesced), already updated by the first
  // sample (index 0) exactly as a visit would: min(d, init), or 0 for a point
  // that does not take part
  const T p0x = P[0], p0y = P[1], p0z = P[2];
  for (int64_t k = tid; k < L.np; k += FPS_THREADS) {
    const FpsRec<T> rc = recs[k];
    const T d = sq3((T)(rc.x - p0x), (T)(rc.y - p0y), (T)(rc.z - p0z));  // fps.cu:145
    ts[k] = rc.key ? (d < init ? d : init) : (T)0;                        // fps.cu:146
  }

  // ---- 3. bucket summaries ----
  // Lane l of wave w owns bucket sb = l * 16 + w: buckets adjacent in Hilbert
  // order (hence in space) belong to different waves, so the few buckets a new
  // sample touches are spread over the workgroup instead of queueing in one wave.
  typedef typename FpsCand<T>::type C;
  C* const ctag = nullptr;
  const int sb = lane * FPS_WAVES + w;
  V blo[3], bhi[3];
  C bbest = cand_none(ctag);
  T bx = (T)0, by = (T)0, bz = (T)0;
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    blo[c] = (V)__builtin_inf();
    bhi[c] = (V)-__builtin_inf();
  }
  if (sb < nb) {
    constexpr int U = 8;  // records in flight per step
    for (int i0 = 0; i0 < s_sz; i0 += U) {
    FpsRec<T> rcu[U];
#pragma unroll
    for (int e = 0; e < U; ++e) rcu[e] = recs[sb * s_sz + i0 + e];
#pragma unroll
    for (int e = 0; e < U; ++e) {
      const FpsRec<T> rc = rcu[e];
      const uint32_t mt = rc.key;
      if (mt == 0) continue;
      const T x = rc.x, y = rc.y, z = rc.z;
      blo[0] = x < blo[0] ? (V)x : blo[0];
      blo[1] = y < blo[1] ? (V)y : blo[1];
      blo[2] = z < blo[2] ? (V)z : blo[2];
      bhi[0] = x > bhi[0] ? (V)x : bhi[0];
      bhi[1] = y > bhi[1] ? (V)y : bhi[1];
      bhi[2] = z > bhi[2] ? (V)z : bhi[2];
      const T d0 = sq3((T)(x - p0x), (T)(y - p0y), (T)(z - p0z));
      const C cand = cand_make((V)(d0 < init ? d0 : init), mt, ctag);
      if (cand_gt(cand, bbest)) {
        bbest = cand;
        bx = x;
        by = y;
        bz = z;
      }
    }
    }
  }
  // the wave's best bucket (uniform)
  int wlane;
  C wbest = wave_best_at(bbest, wlane);

  // ---- 4. the sampling loop ----
  T ox = p0x, oy = p0y, oz = p0z;
  if (tid == 0) out[0] = 0;
  int rk = 0;  // wave 0: lane j mod 64 holds the rank of sample j
  // A bucket is visited only when the squared distance from the new sample to
  // its box is at most reach = max(best * (1 + 2 margin), tiny); beyond it the
  // sample is provably farther from every point in the bucket than that
  // point's running minimum (best bounds them all; the margin dwarfs the
  // rounding of both sides).  A bucket without participating points has
  // reach -1 and is never visited.
  const V grow = (V)1 + (V)2 * (V)FpsConst<T>::margin();
  const V tiny = (V)FpsConst<T>::tiny();
  auto reach_of = [&](C c) -> V { return cand_valid(c) ? vmax((V)cand_val(c) * grow, tiny) : (V)-1; };
  V reach = reach_of(bbest);
  for (int j = 1; j < m; ++j) {
    const V o3[3] = {(V)ox, (V)oy, (V)oz};
    V e[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) e[c] = vmax(vmax(blo[c] - o3[c], o3[c] - bhi[c]), (V)0);
    const V lb2 = vfma(e[2], e[2], vfma(e[1], e[1], e[0] * e[0]));
    // the first sample's updates were made while the cloud was set up
    uint64_t tm = j > 1 ? __ballot(lb2 <= reach) : 0;
    bool rereduce = false;  // the best of the wave's best bucket changed
    // Touched buckets are visited NB at a time: every slot's loads are issued
    // first (the rounds below never leave a slot empty; an empty slot would
    // re-read slot 0's bucket), the NB wave reductions are independent
    // straight-line code, and the running-minimum stores come last, so no load
    // or reduction of the batch waits for a store.
    auto visit = [&](auto nbc) {
      constexpr int NB = decltype(nbc)::value;
      int bits[NB];
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        bits[u] = tm ? __builtin_ctzll(tm) : -1;
        tm &= tm ? tm - 1 : 0;
      }
      for (int p0 = 0; p0 < s_sz; p0 += 64) {
        int pos[NB];
        FpsRec<T> rc[NB];
        T t[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
          const int bu = bits[u] >= 0 ? bits[u] : bits[0];
          pos[u] = (bu * FPS_WAVES + w) * s_sz + p0 + lane;
          rc[u] = recs[pos[u]];
          t[u] = ts[pos[u]];
        }
        T t2[NB];
        C cand[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
          const T d = sq3((T)(rc[u].x - ox), (T)(rc[u].y - oy), (T)(rc[u].z - oz));  // fps.cu:145
          t2[u] = d < t[u] ? d : t[u];                                                // fps.cu:146
          cand[u] = cand_make((V)t2[u], rc[u].key, ctag);
        }
        // A bucket's best stays its best unless that point's own running
        // minimum dropped (the others can only drop too), so the reduction
        // runs only then (always for buckets larger than 64 points).
        bool red[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
          const int bu = bits[u] >= 0 ? bits[u] : bits[0];
          const uint32_t bkey = (uint32_t)__builtin_amdgcn_readlane((int)cand_keyword(bbest), bu);
          red[u] = bits[u] >= 0 && (s_sz > 64 || __ballot(rc[u].key == bkey && t2[u] != t[u]) != 0);
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) {
          if (!red[u]) continue;
          int wl;
          const C best = wave_best_at(cand[u], wl);
          const T cx = bcast(rc[u].x, wl), cy = bcast(rc[u].y, wl), cz = bcast(rc[u].z, wl);
          // passes after the first (buckets larger than 64) keep the max
          if (lane == bits[u] && (p0 == 0 || cand_gt(best, bbest))) {
            bbest = best;
            bx = cx;
            by = cy;
            bz = cz;
          }
          rereduce |= bits[u] == wlane;
        }
#pragma unroll
        for (int u = 0; u < NB; ++u)
          if (bits[u] >= 0 && t2[u] != t[u]) ts[pos[u]] = t2[u];
      }
    };
    if (tm) {
      // the visiting waves set the barrier's arrival: let them issue first
      __builtin_amdgcn_s_setprio(3);
      while (tm) {
        const int nt = __builtin_popcountll(tm);
        // rounds of exactly the touched count (an empty slot would cost a
        // whole load and distance pass), 5 at a time beyond that
        if (nt == 1) visit(std::integral_constant<int, 1>{});
        else if (nt == 2) visit(std::integral_constant<int, 2>{});
        else if (nt == 3) visit(std::integral_constant<int, 3>{});
        else if (nt == 4) visit(std::integral_constant<int, 4>{});
        else visit(std::integral_constant<int, 5>{});
      }
      reach = reach_of(bbest);
      __builtin_amdgcn_s_setprio(0);
    }
    if (rereduce) {  // the wave's best bucket changed; otherwise wbest stands
      wbest = wave_best_at(bbest, wlane);
    }
    const int par = j & 1;
    C g;
    int gw;
    WaveBest mine;
    // the lane holding the wave's best publishes it from its own registers;
    // every lane then reads wave (lane mod 16)'s entry
    if constexpr (sizeof(C) == 8) {
      // Packed keys: every wave folds its best into one LDS word with an
      // atomic max; slots rotate over 3 iterations so the reset of the next
      // slot (before this barrier) never races with its readers (before the
      // previous barrier) or its writers (after this barrier).
      if (tid == 0) s_gkey[(j + 1) % 3] = 0;
      if (lane == wlane) {
        atomicMax(&s_gkey[j % 3], (unsigned long long)bbest.k);
        s_wb[par][w] = WaveBest{bbest, bx, by, bz};
      }
      __syncthreads();
      mine = s_wb[par][lane & (FPS_WAVES - 1)];  // issued with the key read
      g = C{s_gkey[j % 3]};
      gw = lane_of(mine.c, g);
    } else {
      if (lane == wlane) s_wb[par][w] = WaveBest{bbest, bx, by, bz};
      __syncthreads();
      mine = s_wb[par][lane & (FPS_WAVES - 1)];
      g = row0_best(mine.c);
      gw = lane_of(mine.c, g);
    }
    // Nothing participates: the reference's index 0 (rank -1 here).  The
    // rank is decoded to an index after the loop, off the critical path.
    const bool gv = cand_valid(g);
    ox = gv ? bcast(mine.x, gw) : p0x;
    oy = gv ? bcast(mine.y, gw) : p0y;
    oz = gv ? bcast(mine.z, gw) : p0z;
    const int r = gv ? (int)cand_rank(g) : -1;
    // wave 0 stores the ranks 64 at a time
    if (w == 0) {
      rk = lane == (j & 63) ? r : rk;
      if ((j & 63) == 63 || j == m - 1) {
        const int jj = (j & ~63) + lane;
        if (jj >= 1 && jj <= j) out[jj] = (int64_t)rk;
      }
    }
  }
  // rank -> point index: rank = bitrev(k mod BS) * per + k / BS
  __syncthreads();
  for (int j = 1 + tid; j < m; j += FPS_THREADS) {
    const int64_t r = out[j];
    int64_t k = 0;
    if (r >= 0) {
      const uint32_t q = (uint32_t)r / (uint32_t)per, rem = (uint32_t)r - q * (uint32_t)per;
      const uint32_t tq = bs_bits ? (__builtin_bitreverse32(q) >> (32 - bs_bits)) : 0u;
      k = (int64_t)tq + (int64_t)rem * bs;
    }
    out[j] = k;
  }
}

}  // namespace
}  // namespace tpo

using namespace tpo;

extern "C" int64_t tpo_fps_workspace_size(int dtype, int64_t B, int64_t N) {
  if (B < 0 || N < 0) return -1;
  if (N == 0 || B == 0) return 0;
  switch (dtype) {
    case TPO_F32: return B * fps_layout<float>(N).stride;
    case TPO_F64: return B * fps_layout<double>(N).stride;
    case TPO_F16: return B * fps_layout<half_t>(N).stride;
    default: set_error(TPO_ERR_DTYPE, "tpo_fps_workspace_size: unsupported dtype %d", dtype); return -1;
  }
}

extern "C" int tpo_fps_fwd(int dtype, const void* points, int64_t B, int64_t N, int64_t nsamples,
                           int64_t* idx, void* workspace, int64_t workspace_bytes, void* stream) {
  if (B < 0 || N < 1 || nsamples < 1 || nsamples > N || N >= ((int64_t)1 << 30) ||
      B >= ((int64_t)1 << 31))
    return set_error(TPO_ERR_ARG, "tpo_fps_fwd: bad sizes B=%lld N=%lld nsamples=%lld",
                     (long long)B, (long long)N, (long long)nsamples);
  if (B == 0) return TPO_OK;
  const int64_t need = tpo_fps_workspace_size(dtype, B, N);
  if (need < 0) return TPO_ERR_DTYPE;
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255))
    return set_error(TPO_ERR_WORKSPACE, "tpo_fps_fwd: workspace needs %lld bytes (256-aligned)",
                     (long long)need);
  // fps.cu:56-60
  int bs = 1, bits = 0;
  while ((int64_t)bs * 2 <= N && bs < 512) {
    bs *= 2;
    ++bits;
  }
  const int per = (int)((N + bs - 1) / bs);
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case TPO_F32:
      hipLaunchKernelGGL(fps_kernel<float>, dim3((unsigned)B), dim3(FPS_THREADS), 0, s,
                         (const float*)points, (int)N, (int)nsamples, bs, bits, per, (char*)workspace, idx);
      break;
    case TPO_F64:
      hipLaunchKernelGGL(fps_kernel<double>, dim3((unsigned)B), dim3(FPS_THREADS), 0, s,
                         (const double*)points, (int)N, (int)nsamples, bs, bits, per, (char*)workspace, idx);
      break;
    case TPO_F16:
      hipLaunchKernelGGL(fps_kernel<half_t>, dim3((unsigned)B), dim3(FPS_THREADS), 0, s,
                         (const half_t*)points, (int)N, (int)nsamples, bs, bits, per, (char*)workspace, idx);
      break;
    default: return set_error(TPO_ERR_DTYPE, "tpo_fps_fwd: unsupported dtype %d", dtype);
  }
  return check_launch("tpo_fps_fwd");
}
