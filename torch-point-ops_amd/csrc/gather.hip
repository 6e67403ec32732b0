// gather.hip -- gather_points forward/backward for gfx950 (HBM-bound).
//
// Forward (replaces gather_points_kernel, fps.cu:63-76): one thread per
// (cloud, sample, group of 8 channels) reads its index once and gathers the
// channels; stores are coalesced along the sample axis.  With many samples
// per row most cache lines of a row hold a sample, so the cost is the lines
// fetched: the workgroups of one (cloud, channel group) are numbered onto one
// XCD (xcd_logical_block), so each line comes from HBM into one L2 once.
// Backward (replaces zeros + gather_points_grad_kernel, fps.cu:79-98,376):
// instead of a full zero-fill followed by scattered atomics, map each position
// to one sample that lands there, then write grad_points in ONE dense,
// coalesced pass (grad_out[b,c,pos] or 0).  The other samples that repeat a
// position are added afterwards with atomics, which is the reference's
// accumulation for duplicates.  For unique indices every value equals the
// reference's 0 + g exactly.  The dense pass stages a block of grad_out rows
// in LDS per workgroup, so its reads are coalesced as well (a row of M values
// up to 64 KB; longer rows read grad_out[b,c,pos] from memory, a line per
// value).  The map is built in LDS a chunk of positions at a time for M <=
// 4096, else in global memory (pos[b, n] = smallest sample j with
// idx[b, j] == n) by two launches before the pass.
// Indices outside [0, N) are ignored (forward writes 0); the reference reads
// out of bounds there.
// knn_gather (replaces the expand + gather + mask of knn/__init__.py:136-183):
// each (cloud, query, neighbour) row copies the neighbour's U values, or zeros
// for slots at or past lengths[n] (the reference's mask, without its
// host-side lengths.min() test); rows of up to 64 bytes are stored through
// LDS, a wave's 64 rows as one contiguous span.
#include <algorithm>

#include "tpo_common.hpp"

#pragma clang fp contract(off)

namespace tpo {

constexpr int GATHER_CGROUP = 8;

template <typename T>
__global__ __launch_bounds__(256) void gather_fwd_kernel(const T* __restrict__ pts,
                                                         const int64_t* __restrict__ idx,
                                                         int64_t B, int64_t C, int64_t N,
                                                         int64_t M, T* __restrict__ out) {
  const int64_t ncg = (C + GATHER_CGROUP - 1) / GATHER_CGROUP;
  const int64_t total = B * ncg * M;
  for (int64_t t = (int64_t)xcd_logical_block(blockIdx.x, gridDim.x) * 256 + threadIdx.x;
       t < total; t += (int64_t)gridDim.x * 256) {
    const int64_t j = t % M;
    const int64_t bc = t / M;
    const int64_t cg = bc % ncg, b = bc / ncg;
    const int64_t a = idx[b * M + j];
    const bool ok = a >= 0 && a < N;
    const int64_t c0 = cg * GATHER_CGROUP;
    const int64_t cn = min((int64_t)GATHER_CGROUP, C - c0);
    T v[GATHER_CGROUP];
#pragma unroll
    for (int c = 0; c < GATHER_CGROUP; ++c)
      v[c] = (c < cn && ok) ? pts[((b * C) + c0 + c) * N + a] : (T)0;
#pragma unroll
    for (int c = 0; c < GATHER_CGROUP; ++c)
      if (c < cn) out[((b * C) + c0 + c) * M + j] = v[c];
  }
}

__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* __restrict__ p, int64_t n,
                                                       int32_t v) {
  // 16-byte stores over the aligned body, single words at the ends
  const int64_t head = std::min<int64_t>(n, (int64_t)((16 - (reinterpret_cast<uintptr_t>(p) & 15)) & 15) / 4);
  const int64_t body = (n - head) / 4;
  const int4 v4 = make_int4(v, v, v, v);
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x, st = (int64_t)gridDim.x * blockDim.x;
  for (int64_t t = t0; t < body; t += st) reinterpret_cast<int4*>(p + head)[t] = v4;
  for (int64_t t = t0; t < head; t += st) p[t] = v;
  for (int64_t t = head + 4 * body + t0; t < n; t += st) p[t] = v;
}

// pos[b, idx[b, j]] = min over j
__global__ __launch_bounds__(256) void gather_inverse_kernel(const int64_t* __restrict__ idx,
                                                             int64_t B, int64_t N, int64_t M,
                                                             int32_t* __restrict__ pos) {
  const int64_t total = B * M;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = t / M, j = t - b * M;
    const int64_t a = idx[t];
    if (a >= 0 && a < N) atomicMin(pos + b * N + a, (int32_t)j);
  }
}

// grad_points[b, c, n] = pos >= 0 ? grad_out[b, c, pos] : 0, one thread per
// (b, n), looping over channels (stores coalesced along n).
template <typename T>
__global__ __launch_bounds__(256) void gather_bwd_dense_kernel(const T* __restrict__ go,
                                                               const int32_t* __restrict__ pos,
                                                               int64_t B, int64_t C, int64_t N,
                                                               int64_t M, T* __restrict__ gp) {
  const int64_t total = B * N;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = t / N, n = t - b * N;
    const int32_t p = pos[t];
    const bool hit = p != 0x7fffffff;
    const T* __restrict__ src = go + b * C * M + (hit ? p : 0);
    T* __restrict__ dst = gp + b * C * N + n;
    // 0 + g, as the reference's atomicAdd into zeros gives (+0 for g = -0).
    // The empty asm keeps the adds after all four (conditional) loads: left
    // alone, the compiler moves each add into its load's branch, where it
    // waits for that load before the next one is issued.
    int64_t c = 0;
    for (; c + 4 <= C; c += 4) {
      T v0 = hit ? src[(c + 0) * M] : (T)0;
      T v1 = hit ? src[(c + 1) * M] : (T)0;
      T v2 = hit ? src[(c + 2) * M] : (T)0;
      T v3 = hit ? src[(c + 3) * M] : (T)0;
      asm volatile("" : "+v"(v0), "+v"(v1), "+v"(v2), "+v"(v3));
      dst[(c + 0) * N] = (T)((T)0 + v0);
      dst[(c + 1) * N] = (T)((T)0 + v1);
      dst[(c + 2) * N] = (T)((T)0 + v2);
      dst[(c + 3) * N] = (T)((T)0 + v3);
    }
    for (; c < C; ++c) dst[c * N] = hit ? (T)((T)0 + src[c * M]) : (T)0;
  }
}

// The same dense pass with coalesced reads: workgroup (b, channel block,
// part) copies the block's CB rows of grad_out (CB * M contiguous values) into
// LDS, then writes grad_points[b, c, n] for its part of the positions, reading
// grad_out[b, c, pos] from LDS, and adds the repeated samples of those
// positions.  The dense kernel above instead reads each hit's C values from C
// different rows of memory (a line per value).
constexpr int GATHER_ROWS_LDS = 65536;  // LDS bytes for the staged rows
// Workgroups sharing one channel block of a cloud (each stages the rows and
// takes a part of the positions): 2 measured best at config 4.  With the
// position map in global memory: 59 us for the whole backward, 65 with 4, 85
// with 8; 128 KB rows: 69 us with one part.  With the chunked map in LDS:
// 45 us, 57 with 4 parts, 55 with 2-channel blocks (3 workgroups a CU).
constexpr int GATHER_ROWS_PARTS = 2;
constexpr int GATHER_ROWS_THREADS = 1024;
constexpr int GATHER_ROWS_UN = 4;  // positions per thread and step (independent loads)
// LMAP: the part's positions are taken GATHER_MAP_CHUNK at a time, each
// chunk with a position map in LDS (16-bit sample numbers, 0xffff for none)
// built from the thread's GATHER_MAP_JR samples held in registers (M <=
// GATHER_MAP_JR * 1024), so the backward needs no fill and no inverse launch,
// and 64 KB of rows + 16 KB of map let two workgroups share a CU.  The map
// takes the sample of any one plain store among those sharing a position; the
// others are added with atomics, as with the global map.
constexpr int64_t GATHER_MAP_CHUNK = 8192;
constexpr int GATHER_MAP_JR = 4;
template <typename T, int CB, bool LMAP>
__global__ __launch_bounds__(GATHER_ROWS_THREADS) void gather_bwd_rows_kernel(
    const T* __restrict__ go, const int64_t* __restrict__ idx, const int32_t* __restrict__ pos,
    int64_t B, int64_t C, int64_t N, int64_t M, int parts, int64_t map_off,
    T* __restrict__ gp) {
  extern __shared__ __align__(16) unsigned char g_rows[];
  T* __restrict__ rows = reinterpret_cast<T*>(g_rows);
  constexpr int NT = GATHER_ROWS_THREADS, UN = GATHER_ROWS_UN;
  // the parts of one (cloud, channel block) run on one XCD, so its rows come
  // from HBM once
  const int64_t lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int64_t ncb = (C + CB - 1) / CB;
  const int64_t part = lb % parts, bc = lb / parts;
  if (bc >= B * ncb) return;  // the grid's padding to a multiple of 8
  const int64_t cbi = bc % ncb, b = bc / ncb;
  const int64_t c0 = cbi * CB;
  const int cn = (int)min((int64_t)CB, C - c0);
  const T* __restrict__ src = go + (b * C + c0) * M;  // cn rows, contiguous
  const int64_t cnt = (int64_t)cn * M;
  const int64_t vec = (reinterpret_cast<uintptr_t>(src) & 15) == 0 ? cnt * (int64_t)sizeof(T) / 16 : 0;
  for (int64_t i = threadIdx.x; i < vec; i += NT)
    reinterpret_cast<uint4*>(rows)[i] = reinterpret_cast<const uint4*>(src)[i];
  for (int64_t i = vec * 16 / (int64_t)sizeof(T) + threadIdx.x; i < cnt; i += NT) rows[i] = src[i];
  const int64_t n0 = N * part / parts, n1 = N * (part + 1) / parts;
  const int32_t* __restrict__ pb = pos + b * N;
  const int64_t* __restrict__ ib = idx + b * M;
  T* __restrict__ dst = gp + (b * C + c0) * N;
  if constexpr (LMAP) {
    uint16_t* __restrict__ lmap = reinterpret_cast<uint16_t*>(g_rows + map_off);
    constexpr int JR = GATHER_MAP_JR;
    int64_t aj[JR];
    bool rep[JR];  // the sample repeats a position another sample's store takes
#pragma unroll
    for (int r = 0; r < JR; ++r) {
      const int64_t j = threadIdx.x + (int64_t)NT * r;
      aj[r] = j < M ? ib[j] : -1;
      rep[r] = false;
    }
    for (int64_t cs = n0; cs < n1; cs += GATHER_MAP_CHUNK) {
      const int64_t ce = min(cs + GATHER_MAP_CHUNK, n1);
      for (int i = threadIdx.x; i < GATHER_MAP_CHUNK / 8; i += NT)
        reinterpret_cast<uint4*>(lmap)[i] = make_uint4(~0u, ~0u, ~0u, ~0u);
      __syncthreads();  // (first chunk: the rows are staged too)
#pragma unroll
      for (int r = 0; r < JR; ++r)
        if (aj[r] >= cs && aj[r] < ce) lmap[aj[r] - cs] = (uint16_t)(threadIdx.x + NT * r);
      __syncthreads();
#pragma unroll
      for (int r = 0; r < JR; ++r)
        if (aj[r] >= cs && aj[r] < ce)
          rep[r] = lmap[aj[r] - cs] != (uint16_t)(threadIdx.x + NT * r);
      for (int64_t nb = cs + threadIdx.x; nb < ce; nb += (int64_t)NT * UN) {
        int32_t p[UN];
#pragma unroll
        for (int u = 0; u < UN; ++u) {
          const int64_t n = nb + (int64_t)NT * u;
          p[u] = n < ce ? (int32_t)lmap[n - cs] : 0xffff;
        }
#pragma unroll
        for (int u = 0; u < UN; ++u) {
          const int64_t n = nb + (int64_t)NT * u;
          if (n >= ce) break;
          const bool hit = p[u] != 0xffff;
          const T* __restrict__ r = rows + (hit ? p[u] : 0);
          // 0 + g, as the reference's atomicAdd into zeros gives (+0 for g = -0)
#pragma unroll
          for (int c = 0; c < CB; ++c)
            if (c < cn) dst[c * N + n] = hit ? (T)((T)0 + r[c * M]) : (T)0;
        }
      }
      __syncthreads();  // the next chunk's fill waits for this chunk's map reads
    }
    // repeated samples, added once every plain store of the part is done (the
    // last barrier above)
#pragma unroll
    for (int r = 0; r < JR; ++r) {
      if (!rep[r]) continue;
      const int64_t a = aj[r], j = threadIdx.x + (int64_t)NT * r;
#pragma unroll
      for (int c = 0; c < CB; ++c)
        if (c < cn) atomic_add(dst + c * N + a, rows[c * M + j]);
    }
    return;
  }
  __syncthreads();
  for (int64_t nb = n0 + threadIdx.x; nb < n1; nb += (int64_t)NT * UN) {
    int32_t p[UN];
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const int64_t n = nb + (int64_t)NT * u;
      p[u] = n < n1 ? pb[n] : 0x7fffffff;
    }
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const int64_t n = nb + (int64_t)NT * u;
      if (n >= n1) break;
      const bool hit = p[u] != 0x7fffffff;
      const T* __restrict__ r = rows + (hit ? p[u] : 0);
      // 0 + g, as the reference's atomicAdd into zeros gives (+0 for g = -0)
#pragma unroll
      for (int c = 0; c < CB; ++c)
        if (c < cn) dst[c * N + n] = hit ? (T)((T)0 + r[c * M]) : (T)0;
    }
  }
  // Samples that repeat an earlier sample's index, within this part's
  // positions: added with atomics (the reference's accumulation) once the
  // workgroup's own writes of those positions are done.
  __syncthreads();
  for (int64_t j = threadIdx.x; j < M; j += NT) {
    const int64_t a = ib[j];
    if (a < n0 || a >= n1 || pb[a] == (int32_t)j) continue;
#pragma unroll
    for (int c = 0; c < CB; ++c)
      if (c < cn) atomic_add(dst + c * N + a, rows[c * M + j]);
  }
}

// samples whose index repeats an earlier sample's: atomic add
template <typename T>
__global__ __launch_bounds__(256) void gather_bwd_dup_kernel(const T* __restrict__ go,
                                                             const int64_t* __restrict__ idx,
                                                             const int32_t* __restrict__ pos,
                                                             int64_t B, int64_t C, int64_t N,
                                                             int64_t M, T* __restrict__ gp) {
  const int64_t total = B * M;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = t / M, j = t - b * M;
    const int64_t a = idx[t];
    if (a < 0 || a >= N) continue;
    if (pos[b * N + a] == (int32_t)j) continue;
    for (int64_t c = 0; c < C; ++c) atomic_add(gp + (b * C + c) * N + a, go[(b * C + c) * M + j]);
  }
}

// E: an unsigned type of the element's size (the values are only copied).
// One row (n, l, k) a lane, 64 consecutive rows a wave.  TR (rows of at most
// 64 bytes): the wave's rows go through LDS, so its stores cover the 64 * U
// contiguous output values one word a lane, instead of a lane's U values at a
// stride of U words (one row a lane that way touched U times as many lines
// per store).  fp32 rows of 3 values are read with one 12-byte load: at 8 x
// 16384 x 16 rows, 14.5 us against 27.9 with three 4-byte loads (each its own
// line request) and 29.7 without LDS.  I32: total < 2^32, so a row's cloud
// and slot come from 32-bit divisions.
template <typename E, bool I32, bool TR>
__global__ __launch_bounds__(256) void knn_gather_kernel(const E* __restrict__ x,
                                                         const int64_t* __restrict__ idx,
                                                         const int64_t* __restrict__ lengths,
                                                         int64_t N, int64_t M, int64_t L,
                                                         int64_t K, int64_t U,
                                                         E* __restrict__ out) {
  extern __shared__ __align__(16) unsigned char kg_lds[];
  const int64_t total = N * L * K;
  const int lane = threadIdx.x & 63;
  E* __restrict__ wl = reinterpret_cast<E*>(kg_lds) + (threadIdx.x >> 6) * 64 * U;
  for (int64_t tb = (int64_t)blockIdx.x * 256 + (threadIdx.x & ~63); tb < total;
       tb += (int64_t)gridDim.x * 256) {
    const int64_t t = tb + lane;
    int64_t base = -1;  // element offset of the row's source point, -1: zeros
    if (t < total) {
      const int64_t j = idx[t];
      int64_t n, k;
      if constexpr (I32) {
        n = (uint32_t)t / (uint32_t)(L * K);
        k = (uint32_t)t % (uint32_t)K;
      } else {
        n = t / (L * K);
        k = t % K;
      }
      if (k < lengths[n] && j >= 0 && j < M) base = (n * M + j) * U;
    }
    if constexpr (TR) {
      if (sizeof(E) == 4 && U == 3) {  // 3-D points: one 12-byte load a row
        typedef uint32_t w3 __attribute__((ext_vector_type(3), aligned(4)));
        w3 v = {0u, 0u, 0u};
        if (base >= 0) v = *reinterpret_cast<const w3*>(x + base);
        wl[lane * 3 + 0] = (E)v.x;
        wl[lane * 3 + 1] = (E)v.y;
        wl[lane * 3 + 2] = (E)v.z;
      } else {
        for (int64_t u = 0; u < U; ++u) wl[lane * U + u] = base >= 0 ? x[base + u] : (E)0;
      }
      // the wave's LDS writes before its reads of other lanes' rows
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int64_t span = min((int64_t)64, total - tb) * U;
      for (int64_t i = lane; i < span; i += 64) out[tb * U + i] = wl[i];
      // the reads before the next span's writes
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    } else if (t < total) {
      for (int64_t u = 0; u < U; ++u) out[t * U + u] = base >= 0 ? x[base + u] : (E)0;
    }
  }
}

static unsigned grid_for(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 1 << 20) g = 1 << 20;
  return (unsigned)(g < 1 ? 1 : g);
}

// Grid for the XCD-numbered kernels: a multiple of 8 (the XCD count) so that
// xcd_logical_block applies; surplus workgroups find no work.
static unsigned grid_for_xcd(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 1 << 20) g = 1 << 20;
  g = (g + 7) & ~(int64_t)7;
  return (unsigned)(g < 8 ? 8 : g);
}

template <typename T>
static void fwd(const void* pts, const int64_t* idx, int64_t B, int64_t C, int64_t N, int64_t M,
                void* out, hipStream_t s) {
  const int64_t total = B * ((C + GATHER_CGROUP - 1) / GATHER_CGROUP) * M;
  hipLaunchKernelGGL(gather_fwd_kernel<T>, dim3(grid_for_xcd(total)), dim3(256), 0, s,
                     (const T*)pts, idx, B, C, N, M, (T*)out);
}

template <typename T>
static void bwd(const void* go, const int64_t* idx, int64_t B, int64_t C, int64_t N, int64_t M,
                void* gp, int32_t* pos, hipStream_t s) {
  // rows of cb channels staged in LDS where one row fits, else the dense pass
  const int64_t rowb = std::max<int64_t>(1, M * (int64_t)sizeof(T));
  int cb = 1;
  while (cb < 16 && cb < C && 2 * cb * rowb <= GATHER_ROWS_LDS) cb *= 2;
  const int64_t groups = B * ((C + cb - 1) / cb);
  const bool rows = M > 0 && rowb <= GATHER_ROWS_LDS && groups * GATHER_ROWS_PARTS < (1 << 24);
  // the position map in LDS beside the rows, a chunk at a time
  const bool lmap = rows && M <= (int64_t)GATHER_MAP_JR * GATHER_ROWS_THREADS;
  if (!lmap) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3(grid_for((B * N + 3) / 4)), dim3(256), 0, s, pos,
                       B * N, (int32_t)0x7fffffff);
    if (M > 0)
      hipLaunchKernelGGL(gather_inverse_kernel, dim3(grid_for(B * M)), dim3(256), 0, s, idx, B, N,
                         M, pos);
  }
  if (rows) {
    const dim3 g((unsigned)((groups * GATHER_ROWS_PARTS + 7) & ~(int64_t)7));
    const dim3 blk(GATHER_ROWS_THREADS);
    const int64_t map_off = (cb * rowb + 15) / 16 * 16;
    const unsigned lds = (unsigned)(lmap ? map_off + GATHER_MAP_CHUNK * 2 : cb * rowb);
#define GATHER_ROWS(CBV)                                                                        \
  do {                                                                                          \
    if (lmap)                                                                                   \
      hipLaunchKernelGGL((gather_bwd_rows_kernel<T, CBV, true>), g, blk, lds, s, (const T*)go,  \
                         idx, pos, B, C, N, M, GATHER_ROWS_PARTS, map_off, (T*)gp);             \
    else                                                                                        \
      hipLaunchKernelGGL((gather_bwd_rows_kernel<T, CBV, false>), g, blk, lds, s, (const T*)go, \
                         idx, pos, B, C, N, M, GATHER_ROWS_PARTS, map_off, (T*)gp);             \
  } while (0)
    switch (cb) {
      case 1: GATHER_ROWS(1); break;
      case 2: GATHER_ROWS(2); break;
      case 4: GATHER_ROWS(4); break;
      case 8: GATHER_ROWS(8); break;
      default: GATHER_ROWS(16); break;
    }
#undef GATHER_ROWS
  } else {
    hipLaunchKernelGGL(gather_bwd_dense_kernel<T>, dim3(grid_for(B * N)), dim3(256), 0, s,
                       (const T*)go, pos, B, C, N, M, (T*)gp);
    if (M > 0)
      hipLaunchKernelGGL(gather_bwd_dup_kernel<T>, dim3(grid_for(B * M)), dim3(256), 0, s,
                         (const T*)go, idx, pos, B, C, N, M, (T*)gp);
  }
}

}  // namespace tpo

using namespace tpo;

extern "C" int tpo_gather_fwd(int dtype, const void* points, const int64_t* idx, int64_t B,
                              int64_t C, int64_t N, int64_t M, void* out, void* stream) {
  if (B < 0 || C < 0 || N < 0 || M < 0)
    return set_error(TPO_ERR_ARG, "tpo_gather_fwd: negative size");
  if (B == 0 || C == 0 || M == 0) return TPO_OK;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case TPO_F32: fwd<float>(points, idx, B, C, N, M, out, s); break;
    case TPO_F64: fwd<double>(points, idx, B, C, N, M, out, s); break;
    case TPO_F16: fwd<half_t>(points, idx, B, C, N, M, out, s); break;
    default: return set_error(TPO_ERR_DTYPE, "tpo_gather_fwd: unsupported dtype %d", dtype);
  }
  return check_launch("tpo_gather_fwd");
}

extern "C" int64_t tpo_gather_bwd_workspace_size(int64_t B, int64_t N) {
  if (B < 0 || N < 0) return -1;
  return ((B * N * 4 + 255) / 256) * 256;
}

extern "C" int tpo_gather_bwd(int dtype, const void* grad_out, const int64_t* idx, int64_t B,
                              int64_t C, int64_t N, int64_t M, void* grad_points, void* workspace,
                              int64_t workspace_bytes, void* stream) {
  if (B < 0 || C < 0 || N < 0 || M < 0 || N >= ((int64_t)1 << 31) || M >= ((int64_t)1 << 31))
    return set_error(TPO_ERR_ARG, "tpo_gather_bwd: bad sizes");
  if (B == 0 || C == 0 || N == 0) return TPO_OK;
  if (!workspace || workspace_bytes < B * N * 4)
    return set_error(TPO_ERR_WORKSPACE, "tpo_gather_bwd: workspace of %lld bytes < %lld",
                     (long long)workspace_bytes, (long long)(B * N * 4));
  hipStream_t s = (hipStream_t)stream;
  int32_t* pos = (int32_t*)workspace;
  switch (dtype) {
    case TPO_F32: bwd<float>(grad_out, idx, B, C, N, M, grad_points, pos, s); break;
    case TPO_F64: bwd<double>(grad_out, idx, B, C, N, M, grad_points, pos, s); break;
    case TPO_F16: bwd<half_t>(grad_out, idx, B, C, N, M, grad_points, pos, s); break;
    default: return set_error(TPO_ERR_DTYPE, "tpo_gather_bwd: unsupported dtype %d", dtype);
  }
  return check_launch("tpo_gather_bwd");
}

extern "C" int tpo_knn_gather(int dtype, const void* x, const int64_t* idx,
                              const int64_t* lengths, int64_t N, int64_t M, int64_t L, int64_t K,
                              int64_t U, void* out, void* stream) {
  if (N < 0 || M < 0 || L < 0 || K < 0 || U < 0)
    return set_error(TPO_ERR_ARG, "tpo_knn_gather: negative size");
  if (N == 0 || L == 0 || K == 0 || U == 0) return TPO_OK;
  if (M == 0) return set_error(TPO_ERR_ARG, "tpo_knn_gather: x has no points");
  hipStream_t s = (hipStream_t)stream;
  const int64_t total = N * L * K;
  const unsigned g = grid_for(total);
  const bool i32 = total <= (int64_t)UINT32_MAX;
#define KNN_GATHER_L(E, I, TRV)                                                               \
  hipLaunchKernelGGL((knn_gather_kernel<E, I, TRV>), dim3(g), dim3(256),                     \
                     TRV ? (unsigned)(256 * U * sizeof(E)) : 0u, s, (const E*)x, idx, lengths, \
                     N, M, L, K, U, (E*)out)
#define KNN_GATHER(E)                                                       \
  do {                                                                      \
    const bool tr = U * (int64_t)sizeof(E) <= 64;                           \
    if (i32 && tr) KNN_GATHER_L(E, true, true);                             \
    else if (i32) KNN_GATHER_L(E, true, false);                             \
    else if (tr) KNN_GATHER_L(E, false, true);                              \
    else KNN_GATHER_L(E, false, false);                                     \
  } while (0)
  switch (dtype) {
    case TPO_F32: KNN_GATHER(uint32_t); break;
    case TPO_F64: KNN_GATHER(uint64_t); break;
    case TPO_F16:
    case TPO_BF16: KNN_GATHER(uint16_t); break;
    default: return set_error(TPO_ERR_DTYPE, "tpo_knn_gather: unsupported dtype %d", dtype);
  }
#undef KNN_GATHER
#undef KNN_GATHER_L
  return check_launch("tpo_knn_gather");
}
