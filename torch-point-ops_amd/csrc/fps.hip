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
//   1. The workgroup sorts its cloud into a workspace by Morton cell of a
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
//   sample, while the result is bit-identical to the full sweep.
#include "tpo_common.hpp"

#pragma clang fp contract(off)

namespace tpo {
namespace {

constexpr int FPS_THREADS = 1024;
constexpr int FPS_WAVES = FPS_THREADS / 64;
constexpr int FPS_GRID = 16;  // Morton grid per axis (4096 cells)
constexpr int FPS_CELLS = FPS_GRID * FPS_GRID * FPS_GRID;
constexpr uint32_t FPS_INVALID = 0x80000000u;

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

struct FpsLayout {
  int64_t np;      // padded points per cloud = nb * s
  int64_t stride;  // bytes per cloud
  int64_t off_x, off_y, off_z, off_t, off_m;
};

template <typename T>
__host__ __device__ inline FpsLayout fps_layout(int64_t n) {
  const int64_t s = 64 * ((n + 64 * FPS_THREADS - 1) / (64 * FPS_THREADS));
  const int64_t nb = (n + s - 1) / s;
  FpsLayout L;
  L.np = nb * s;
  auto al = [](int64_t v) { return (v + 255) / 256 * 256; };
  int64_t o = 0;
  L.off_x = o; o += al(L.np * (int64_t)sizeof(T));
  L.off_y = o; o += al(L.np * (int64_t)sizeof(T));
  L.off_z = o; o += al(L.np * (int64_t)sizeof(T));
  L.off_t = o; o += al(L.np * (int64_t)sizeof(T));
  L.off_m = o; o += al(L.np * 4);
  L.stride = o;
  return L;
}

__device__ __forceinline__ uint32_t spread3(uint32_t v) {  // 4 bits -> every third bit
  v &= 0xf;
  v = (v | (v << 4)) & 0x0c3;
  v = (v | (v << 2)) & 0x249;
  return v;
}

template <typename V>
__device__ __forceinline__ bool better(V va, uint32_t ra, V vb, uint32_t rb) {
  return va > vb || (va == vb && ra < rb);
}

template <typename V>
__device__ __forceinline__ V shfl_xor_v(V v, int m) { return __shfl_xor(v, m, 64); }

// Reduce (val, rank) to the wave's best; returns the best lane's values in
// every lane and the index of (one) lane holding it.
template <typename V>
__device__ __forceinline__ int wave_best(V& val, uint32_t& rank) {
  V bv = val;
  uint32_t br = rank;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const V ov = shfl_xor_v(bv, m);
    const uint32_t orr = (uint32_t)__shfl_xor((int)br, m, 64);
    if (better(ov, orr, bv, br)) {
      bv = ov;
      br = orr;
    }
  }
  const uint64_t hit = __ballot(val == bv && rank == br);
  val = bv;
  rank = br;
  return hit ? __builtin_ctzll(hit) : 0;
}

__device__ __forceinline__ float bcast(float v, int lane) { return __shfl(v, lane, 64); }
__device__ __forceinline__ double bcast(double v, int lane) { return __shfl(v, lane, 64); }
__device__ __forceinline__ half_t bcast(half_t v, int lane) {
  return (half_t)__shfl((float)v, lane, 64);  // exact round trip
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
  __shared__ V s_bv[2][FPS_WAVES];
  __shared__ uint32_t s_br[2][FPS_WAVES];
  __shared__ T s_bx[2][FPS_WAVES], s_by[2][FPS_WAVES], s_bz[2][FPS_WAVES];

  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
  const FpsLayout L = fps_layout<T>(N);
  const int s_sz = (int)(64 * ((N + 64 * FPS_THREADS - 1) / (64 * FPS_THREADS)));
  const int nb = (N + s_sz - 1) / s_sz;
  char* base = ws + (size_t)b * L.stride;
  T* __restrict__ xs = (T*)(base + L.off_x);
  T* __restrict__ ys = (T*)(base + L.off_y);
  T* __restrict__ zs = (T*)(base + L.off_z);
  T* __restrict__ ts = (T*)(base + L.off_t);
  uint32_t* __restrict__ ms = (uint32_t*)(base + L.off_m);
  const T* __restrict__ P = pts + (size_t)b * N * 3;
  int64_t* __restrict__ out = idx_out + (size_t)b * m;

  // ---- 1. bounding box of the cloud (for the Morton grid only) ----
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

  // ---- 2. counting sort by Morton cell ----
  auto cell_of = [&](int k) -> uint32_t {
    uint32_t cc[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      float f = ((float)P[3 * k + c] - glo[c]) * gscale[c];
      int i = (f == f) ? (int)f : 0;
      i = i < 0 ? 0 : (i > FPS_GRID - 1 ? FPS_GRID - 1 : i);
      cc[c] = (uint32_t)i;
    }
    return spread3(cc[0]) | (spread3(cc[1]) << 1) | (spread3(cc[2]) << 2);
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
    xs[pos] = x;
    ys[pos] = y;
    zs[pos] = z;
    ts[pos] = init;
    ms[pos] = rank | (valid ? 0u : FPS_INVALID);
  }
  for (int64_t k = N + tid; k < L.np; k += FPS_THREADS) {
    xs[k] = (T)0;
    ys[k] = (T)0;
    zs[k] = (T)0;
    ts[k] = (T)0;
    ms[k] = FPS_INVALID;
  }
  __syncthreads();

  // ---- 3. bucket summaries: lane owns bucket sb = w*64 + lane ----
  const int sb = w * 64 + lane;
  V blo[3], bhi[3];
  V bval = (V)-1;
  uint32_t brank = 0xffffffffu;
  T bx = (T)0, by = (T)0, bz = (T)0;
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    blo[c] = (V)__builtin_inf();
    bhi[c] = (V)-__builtin_inf();
  }
  if (sb < nb) {
    for (int i = 0; i < s_sz; ++i) {
      const int pos = sb * s_sz + i;
      const uint32_t mt = ms[pos];
      if (mt & FPS_INVALID) continue;
      const T x = xs[pos], y = ys[pos], z = zs[pos];
      blo[0] = x < blo[0] ? (V)x : blo[0];
      blo[1] = y < blo[1] ? (V)y : blo[1];
      blo[2] = z < blo[2] ? (V)z : blo[2];
      bhi[0] = x > bhi[0] ? (V)x : bhi[0];
      bhi[1] = y > bhi[1] ? (V)y : bhi[1];
      bhi[2] = z > bhi[2] ? (V)z : bhi[2];
      if (better((V)init, mt, bval, brank)) {
        bval = (V)init;
        brank = mt;
        bx = x;
        by = y;
        bz = z;
      }
    }
  }

  // ---- 4. the sampling loop ----
  T ox = P[0], oy = P[1], oz = P[2];
  if (tid == 0) out[0] = 0;
  const V margin = (V)FpsConst<T>::margin();
  const V tiny = (V)FpsConst<T>::tiny();
  for (int j = 1; j < m; ++j) {
    bool touch = false;
    if (bval >= (V)0) {
      V lb2 = (V)0;
      const V o3[3] = {(V)ox, (V)oy, (V)oz};
#pragma unroll
      for (int c = 0; c < 3; ++c) {
        V e = blo[c] - o3[c];
        const V f = o3[c] - bhi[c];
        e = e > f ? e : f;
        e = e > (V)0 ? e : (V)0;
        lb2 += e * e;
      }
      touch = !(lb2 * ((V)1 - margin) > bval && lb2 > tiny);
    }
    uint64_t tm = __ballot(touch);
    while (tm) {
      const int bit = __builtin_ctzll(tm);
      tm &= tm - 1;
      const int bk = w * 64 + bit;
      V cv = (V)-1;
      uint32_t cr = 0xffffffffu;
      T cx = (T)0, cy = (T)0, cz = (T)0;
      for (int p0 = 0; p0 < s_sz; p0 += 64) {
        const int pos = bk * s_sz + p0 + lane;
        const uint32_t mt = ms[pos];
        if (!(mt & FPS_INVALID)) {
          const T x = xs[pos], y = ys[pos], z = zs[pos];
          const T t = ts[pos];
          const T d = sq3((T)(x - ox), (T)(y - oy), (T)(z - oz));  // fps.cu:145
          const T t2 = d < t ? d : t;                                // fps.cu:146
          if (t2 != t) ts[pos] = t2;
          if (better((V)t2, mt, cv, cr)) {
            cv = (V)t2;
            cr = mt;
            cx = x;
            cy = y;
            cz = z;
          }
        }
      }
      const int wl = wave_best(cv, cr);
      cx = bcast(cx, wl);
      cy = bcast(cy, wl);
      cz = bcast(cz, wl);
      if (lane == bit) {
        bval = cv;
        brank = cr;
        bx = cx;
        by = cy;
        bz = cz;
      }
    }
    // wave best over its buckets, then the workgroup best
    V wv = bval;
    uint32_t wr = brank;
    const int wl = wave_best(wv, wr);
    const T wx = bcast(bx, wl), wy = bcast(by, wl), wz = bcast(bz, wl);
    const int par = j & 1;
    if (lane == 0) {
      s_bv[par][w] = wv;
      s_br[par][w] = wr;
      s_bx[par][w] = wx;
      s_by[par][w] = wy;
      s_bz[par][w] = wz;
    }
    __syncthreads();
    V gv = s_bv[par][0];
    uint32_t gr = s_br[par][0];
    int gw = 0;
#pragma unroll
    for (int v2 = 1; v2 < FPS_WAVES; ++v2) {
      const V vv = s_bv[par][v2];
      const uint32_t rr = s_br[par][v2];
      if (better(vv, rr, gv, gr)) {
        gv = vv;
        gr = rr;
        gw = v2;
      }
    }
    int64_t k;
    if (gv < (V)0) {  // nothing participates: the reference's index 0
      k = 0;
      ox = P[0];
      oy = P[1];
      oz = P[2];
    } else {
      const uint32_t r = gr & ~FPS_INVALID;
      const uint32_t q = r / (uint32_t)per, rem = r - q * (uint32_t)per;
      const uint32_t t = bs_bits ? (__builtin_bitreverse32(q) >> (32 - bs_bits)) : 0u;
      k = (int64_t)t + (int64_t)rem * bs;
      ox = s_bx[par][gw];
      oy = s_by[par][gw];
      oz = s_bz[par][gw];
    }
    if (tid == 0) out[j] = k;
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
