// knn_grid.hip -- exact K nearest neighbours of float 3-D points against long
// reference clouds (knn_points at config 3's shape), in the reference's MinK
// slot layout (knn.cu:113-168, mink.cuh:77-121).
//
// The MinK process fills its K slots with references 0 .. K-1 and then
// replaces the first slot holding the maximum with every later reference
// that is strictly closer than that maximum; the slot layout depends on the
// whole sequence of such insertions.  Its maximum never increases.  So after
// a prefix [0, A) of the references has been processed exactly, every later
// insertion j satisfies d(j) < T, T being the maximum after the prefix, and
// lies within sqrt(T) of the query on each axis (within T for norm 1).  A
// process that sees the prefix, then every later reference of a superset of
// those in index order, makes the same insertions: whenever it meets a real
// insertion its state equals the real one (induction over the insertions),
// and a reference that is no real insertion is not below the real maximum
// at that point, which is the state's maximum.  The superset here is "every
// reference in the grid cells that a box of half-width B around any query of
// the wave touches", with B a bound on the axis distance that covers the
// rounding of the computed distance; cells are assigned by one monotonic
// function for references and box ends alike.
//
// knn_grid_setup_kernel: per cloud, one workgroup orders the queries (Hilbert
//   order of a 16^3 grid over them, so that a wave's 64 queries are
//   neighbours) and one builds a 16^3 grid over the bounding box of the
//   finite references [0, lengths2): cell start table and the reference
//   indices by cell (any order within a cell).
// knn_grid_kernel: one query per lane, in that order.
//   1. the brute-force prefix over references [K, A) in chunks of 32: each
//      16-lane row loads 16 references and DPP broadcasts them over the row;
//      the chunk's distances go into a candidate mask against the lane's
//      maximum and each lane walks its own candidates in order;
//   2. the wave's box of cells (the union of its lanes' boxes); when it is
//      small, the references >= A in those cells are marked in a wave-private
//      LDS bitmask over reference indices, which is then compacted, 2048
//      indices at a time, into index order and processed like step 1 with
//      the references gathered by index.  A wave with a large box, or a
//      non-finite bound, processes [A, lengths2) by brute force instead.
#include <utility>

#include "knn_common.hpp"

namespace tpo {
namespace {

constexpr int KG_G = 16;                      // grid cells per axis
constexpr int KG_CELLS = KG_G * KG_G * KG_G;
constexpr int KG_WIN = 512;                   // candidates per window (a multiple of 64)
constexpr int KG_MAX_BOX = 4096;              // cells a wave's boxes hold at most before it sweeps
constexpr int KG_WAVES = 4;
constexpr int KG_RING = 3;                    // chunks of coordinates in flight

template <typename F, int... C>
__device__ __forceinline__ void kg_static_for(F&& f, std::integer_sequence<int, C...>) {
  (f(std::integral_constant<int, C>{}), ...);
}

// Grid cell along one axis: monotonic non-decreasing in x (a subtraction, a
// product by gs >= 0, a clamp and a truncation of a non-negative value);
// NaN lands in cell 0.
__device__ __forceinline__ int kg_axis(float x, float lo, float gs) {
  float f = (x - lo) * gs;
  f = fminf(fmaxf(f, 0.f), (float)(KG_G - 1));
  return (int)f;
}


// knn.cu:148-158 for D = 3
template <int NORM>
__device__ __forceinline__ float kg_dist(const float (&q)[3], float x, float y, float z) {
  float a = NORM == 2 ? knn_acc2(0.f, q[0] - x, true) : knn_acc1(0.f, q[0] - x, true);
  a = NORM == 2 ? knn_acc2(a, q[1] - y, false) : knn_acc1(a, q[1] - y, false);
  a = NORM == 2 ? knn_acc2(a, q[2] - z, false) : knn_acc1(a, q[2] - z, false);
  return a;
}

// Points [0, L) of one cloud binned into a 16^3 grid over the bounding box
// of its finite points: HILBERT orders the cells along a Hilbert curve (the
// query processing order: consecutive cells are face neighbours, so the 64
// queries of a wave stay in a compact region), otherwise by (x, y, z)
// row-major (the reference grid, whose cells along z then sit next to each
// other).  Writes the box to hdr and the exclusive cell starts to cs when
// given, and the point indices grouped by cell to out[0, L) (any order
// within a cell).  PPT > 0 (L <= 1024 PPT): each thread's points are loaded
// once into registers, their cells computed once, and placed by the rank
// the histogram's atomics returned; PPT == 0 streams the cloud three times.
struct KgBinLds {
  uint32_t cnt[KG_CELLS];
  float red[6][16];
  uint32_t part[16];
};

template <bool HILBERT, int PPT>
__device__ void kg_bin(const float* __restrict__ P, int L, float* __restrict__ hdr,
                       int32_t* __restrict__ cs, int32_t* __restrict__ out, KgBinLds& sm) {
  uint32_t* __restrict__ cnt = sm.cnt;
  float (*red)[16] = sm.red;
  uint32_t* __restrict__ part = sm.part;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  constexpr int R = PPT > 0 ? PPT : 4;  // points a thread holds at once
  float v[R][3];
  auto load = [&](int k0) {  // points k0 + 1024 u, clamped (a repeat changes no bound)
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int k = min(k0 + 1024 * u, L - 1);
#pragma unroll
      for (int c = 0; c < 3; ++c) v[u][c] = P[3 * k + c];
    }
  };
  float lo[3] = {__builtin_inff(), __builtin_inff(), __builtin_inff()};
  float hi[3] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
  auto bound = [&]() {
#pragma unroll
    for (int u = 0; u < R; ++u)
#pragma unroll
      for (int c = 0; c < 3; ++c)
        if (__builtin_fabsf(v[u][c]) < __builtin_inff()) {
          lo[c] = fminf(lo[c], v[u][c]);
          hi[c] = fmaxf(hi[c], v[u][c]);
        }
  };
  if (L > 0) {
    if constexpr (PPT > 0) {
      load(tid);
      bound();
    } else {
      for (int k0 = tid; k0 < L; k0 += 1024 * R) {
        load(k0);
        bound();
      }
    }
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
  for (int c = tid; c < KG_CELLS; c += 1024) cnt[c] = 0;
  __syncthreads();
  float glo[3], gs[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    float a = __builtin_inff(), z = -__builtin_inff();
    for (int x = 0; x < 16; ++x) {
      a = fminf(a, red[c][x]);
      z = fmaxf(z, red[3 + c][x]);
    }
    const float ext = z - a;
    const bool fin = ext > 0.f && ext < __builtin_inff();
    glo[c] = a < __builtin_inff() ? a : 0.f;  // no finite point: one cell
    gs[c] = fin ? (float)KG_G / ext : 0.f;
  }
  if (hdr && tid < 3) {
    hdr[tid] = glo[tid];
    hdr[3 + tid] = gs[tid];
  }
  auto cell_of = [&](float x, float y, float z) -> int {
    const int ci[3] = {kg_axis(x, glo[0], gs[0]), kg_axis(y, glo[1], gs[1]),
                       kg_axis(z, glo[2], gs[2])};
    if constexpr (HILBERT) {
      return (int)hilbert3_16(ci[0], ci[1], ci[2]);
    } else {
      return (ci[0] * KG_G + ci[1]) * KG_G + ci[2];
    }
  };
  int cell[PPT > 0 ? PPT : 1];
  uint32_t rank[PPT > 0 ? PPT : 1];
  if constexpr (PPT > 0) {  // histogram from registers, ranks kept
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
      const int k = tid + 1024 * u;
      if (k < L) {
        cell[u] = cell_of(v[u][0], v[u][1], v[u][2]);
        rank[u] = atomicAdd(&cnt[cell[u]], 1u);
      }
    }
  } else {  // histogram, then (after the scan) ranks, streaming R points a thread
    for (int k0 = tid; k0 < L; k0 += 1024 * R) {
      load(k0);
#pragma unroll
      for (int u = 0; u < R; ++u)
        if (k0 + 1024 * u < L) atomicAdd(&cnt[cell_of(v[u][0], v[u][1], v[u][2])], 1u);
    }
  }
  __syncthreads();
  {  // exclusive scan, 4 cells per thread
    uint32_t c4[4], sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c4[i] = cnt[tid * 4 + i];
      sum += c4[i];
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
      if (cs) cs[tid * 4 + i] = (int32_t)run;
      run += c4[i];
    }
    if (cs && tid == 0) cs[KG_CELLS] = L;
  }
  __syncthreads();
  if constexpr (PPT > 0) {
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
      const int k = tid + 1024 * u;
      if (k < L) out[cnt[cell[u]] + rank[u]] = k;
    }
  } else {
    for (int k0 = tid; k0 < L; k0 += 1024 * R) {
      load(k0);
#pragma unroll
      for (int u = 0; u < R; ++u) {
        const int k = k0 + 1024 * u;
        if (k < L) out[atomicAdd(&cnt[cell_of(v[u][0], v[u][1], v[u][2])], 1u)] = k;
      }
    }
  }
}

constexpr int KG_PPT = 16;  // register-resident binning up to 16384 points

// Blocks [0, N): the processing order of cloud n's queries (valid rows in
// Hilbert order of their own grid, rows past lengths1 after them in place);
// blocks [N, 2N): the grid of cloud n's references [0, lengths2).
__global__ __launch_bounds__(1024) void knn_grid_setup_kernel(
    const float* __restrict__ p1, const int64_t* __restrict__ len1, int P1,
    int32_t* __restrict__ order, const float* __restrict__ p2, const int64_t* __restrict__ len2,
    int P2, int N, float* __restrict__ hdr, int32_t* __restrict__ cstart,
    int32_t* __restrict__ list) {
  __shared__ KgBinLds sm;
  if ((int)blockIdx.x < N) {
    const int n = blockIdx.x;
    const int64_t l1 = len1[n];
    const int L1 = (int)(l1 < 0 ? 0 : (l1 > P1 ? P1 : l1));
    int32_t* __restrict__ out = order + (size_t)n * P1;
    if (L1 <= 1024 * KG_PPT) kg_bin<true, KG_PPT>(p1 + (size_t)n * P1 * 3, L1, nullptr, nullptr, out, sm);
    else kg_bin<true, 0>(p1 + (size_t)n * P1 * 3, L1, nullptr, nullptr, out, sm);
    for (int k = L1 + (int)threadIdx.x; k < P1; k += 1024) out[k] = k;
  } else {
    const int n = blockIdx.x - N;
    const int64_t l2 = len2[n];
    const int L2 = (int)(l2 < 0 ? 0 : (l2 > P2 ? P2 : l2));
    float* h = hdr + (size_t)n * 8;
    int32_t* cs = cstart + (size_t)n * (KG_CELLS + 1);
    int32_t* ls = list + (size_t)n * P2;
    if (L2 <= 1024 * KG_PPT) kg_bin<false, KG_PPT>(p2 + (size_t)n * P2 * 3, L2, h, cs, ls, sm);
    else kg_bin<false, 0>(p2 + (size_t)n * P2 * 3, L2, h, cs, ls, sm);
  }
}

template <int NORM, int KC, bool SORT>
__global__ __launch_bounds__(256) void knn_grid_kernel(
    const float* __restrict__ p1, const float* __restrict__ p2, const int64_t* __restrict__ len1,
    const int64_t* __restrict__ len2, const int32_t* __restrict__ order,
    const float* __restrict__ hdr, const int32_t* __restrict__ cstart,
    const int32_t* __restrict__ list, int P1, int P2, int K, int A, int nqb, int words,
    int pad_sentinel, int64_t* __restrict__ idxs, float* __restrict__ dists) {
  // LDS per wave: `words` bitmask words, a window of KG_WIN candidate
  // indices, and the current chunk's distances ([entry][lane])
  extern __shared__ uint32_t kg_lds[];
  const int w = wave_id(), lane = lane_id();
  uint32_t* __restrict__ bm = kg_lds + (size_t)w * (words + KG_WIN + KNN_CHUNK * 64);
  int32_t* __restrict__ cl = reinterpret_cast<int32_t*>(bm + words);
  float* __restrict__ dl = reinterpret_cast<float*>(cl + KG_WIN) + lane;
  const int n = blockIdx.x / nqb;
  int64_t l1 = len1[n], l2 = len2[n];
  l1 = l1 < 0 ? 0 : (l1 > P1 ? P1 : l1);
  l2 = l2 < 0 ? 0 : (l2 > P2 ? P2 : l2);
  const int L2 = (int)l2;
  const int Ae = min(A, L2);
  const float* __restrict__ rp = p2 + (size_t)n * P2 * 3;

  const int i = (blockIdx.x - n * nqb) * 256 + threadIdx.x;  // position in processing order
  const bool in_range = i < P1;
  const int q = in_range ? order[(size_t)n * P1 + i] : 0;
  const size_t row = (size_t)n * P1 + q;
  int64_t* __restrict__ io = idxs + row * K;
  float* __restrict__ dout = dists + row * K;
  const bool act = in_range && q < l1;
  if (in_range && !act) {  // never written by the reference: its zeros
    for (int s = 0; s < K; ++s) {
      io[s] = 0;
      dout[s] = 0.f;
    }
  }
  // rows past lengths1 sit at the end of the processing order
  if (__ballot(act) == 0) return;
  float qr[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) qr[c] = act ? p1[row * 3 + c] : 0.f;

  float sd[KC];
  int si[KC];
  const int fill = L2 < K ? L2 : K;
#pragma unroll
  for (int s = 0; s < KC; ++s) {
    if (s < fill) {
      sd[s] = kg_dist<NORM>(qr, rp[3 * s], rp[3 * s + 1], rp[3 * s + 2]);
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
    if (!act) thr = -Lim<float>::inf();  // a lane without a query has no candidates

    // A chunk: up to 32 references, lane l holding the coordinates of chunk
    // entries l % 16 (b = 0) and 16 + l % 16 (b = 1).  Entries past cn are
    // +inf.  The distances go to LDS; mask bit 31 - c flags entry c.
    auto chunk = [&](const float (&bx)[2], const float (&by)[2], const float (&bz)[2], int cn) {
      float dd[KNN_CHUNK];
      kg_static_for(
          [&](auto cc) {
            constexpr int c = decltype(cc)::value;
            float d = kg_dist<NORM>(qr, row_bcast<c % 16>(bx[c / 16]), row_bcast<c % 16>(by[c / 16]),
                                    row_bcast<c % 16>(bz[c / 16]));
            d = c < cn ? d : Lim<float>::inf();
            dl[64 * c] = d;
            dd[c] = d;
          },
          std::make_integer_sequence<int, KNN_CHUNK>{});
      uint32_t mask = 0;
#pragma unroll
      for (int c = 0; c < KNN_CHUNK; c += 4)
        mask = push_lt4(mask, dd[c], dd[c + 1], dd[c + 2], dd[c + 3], thr);
      return mask;
    };
    // this lane's candidates of the chunk in order, against the current
    // maximum; the next candidate's distance is read ahead
    auto walk = [&](uint32_t mask, auto&& index_of) {
      int top = mask ? 31 - __builtin_clz(mask) : 0;
      float dn = dl[64 * (31 - top)];
      while (mask) {
        const int c = 31 - top;
        const float d = dn;
        mask ^= 1u << top;
        top = mask ? 31 - __builtin_clz(mask) : 0;
        dn = dl[64 * (31 - top)];
        if (d < thr) {
          const int j = index_of(c);
          mink_put<float, KC>(sd, si, ms, d, j);
          first_max<float, KC>(sd, K, thr, ms);
        }
      }
    };
    // entries [e_begin, e_end) in chunks of 32, the reference of entry e
    // being ref_of(e); the coordinates of KG_RING chunks are in flight
    auto run = [&](int e_begin, int e_end, auto&& ref_of) {
      float rx[KG_RING][2], ry[KG_RING][2], rz[KG_RING][2];
      auto load = [&](float (&x)[2], float (&y)[2], float (&z)[2], int eb) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const int j = ref_of(min(eb + 16 * b + (lane & 15), e_end - 1));
          x[b] = rp[3 * j];
          y[b] = rp[3 * j + 1];
          z[b] = rp[3 * j + 2];
        }
      };
#pragma unroll
      for (int r = 0; r < KG_RING; ++r) load(rx[r], ry[r], rz[r], e_begin + KNN_CHUNK * r);
      for (int e0 = e_begin; e0 < e_end; e0 += KNN_CHUNK * KG_RING) {
#pragma unroll
        for (int r = 0; r < KG_RING; ++r) {
          const int eb = e0 + KNN_CHUNK * r;
          if (eb < e_end) {
            const uint32_t mask = chunk(rx[r], ry[r], rz[r], min(KNN_CHUNK, e_end - eb));
            load(rx[r], ry[r], rz[r], eb + KNN_CHUNK * KG_RING);
            walk(mask, [&](int c) { return ref_of(eb + c); });
          }
        }
      }
    };
    // the prefix [K, Ae)
    run(K, Ae, [](int e) { return e; });
    if (L2 > Ae) {
      // the lane's box: every later insertion is within B of the query per axis
      const float* __restrict__ h = hdr + (size_t)n * 8;
      int blo[3], bhi[3];
      bool ok = true;
      if (act) {
        float B;
        if (NORM == 2) B = __builtin_sqrtf(thr + 0x1p-120f) * (1.f + 0x1p-18f) + 0x1p-60f;
        else B = thr * (1.f + 0x1p-18f) + 0x1p-100f;
        ok = B < Lim<float>::inf();
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          const float Bc = B + (__builtin_fabsf(qr[c]) + B) * 0x1p-20f;
          ok = ok && __builtin_fabsf(qr[c]) < Lim<float>::inf();
          blo[c] = kg_axis(qr[c] - Bc, h[c], h[3 + c]);
          bhi[c] = kg_axis(qr[c] + Bc, h[c], h[3 + c]);
        }
      } else {
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          blo[c] = KG_G;
          bhi[c] = -1;
        }
      }
      // one box per 16-lane row (the union of its lanes' boxes): a wave that
      // straddles a jump of the query order keeps four compact boxes
#pragma unroll
      for (int c = 0; c < 3; ++c)
#pragma unroll
        for (int m = 8; m >= 1; m >>= 1) {
          blo[c] = min(blo[c], __shfl_xor(blo[c], m, 64));
          bhi[c] = max(bhi[c], __shfl_xor(bhi[c], m, 64));
        }
      const int ex = bhi[0] - blo[0] + 1, ey = bhi[1] - blo[1] + 1, ez = bhi[2] - blo[2] + 1;
      const bool nonempty = ex > 0 && ey > 0 && ez > 0;  // the row has a query
      const int rcells = nonempty ? ex * ey * ez : 0, rruns = nonempty ? ex * ey : 0;
      int cells = 0, runs_pre[5];
      runs_pre[0] = 0;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        cells += __shfl(rcells, 16 * g, 64);
        runs_pre[g + 1] = runs_pre[g] + __shfl(rruns, 16 * g, 64);
      }
      const int w0 = Ae >> 5, w1 = (L2 + 31) >> 5;
      if (__ballot(!ok) != 0 || cells > KG_MAX_BOX) {
        // no useful box: every reference of [Ae, L2) is a candidate
        for (int t = w0 + lane; t < w1; t += 64) {
          const int b0 = max(Ae - 32 * t, 0), b1 = min(L2 - 32 * t, 32);
          bm[t] = (b1 >= 32 ? 0xffffffffu : (1u << b1) - 1u) & ~((1u << b0) - 1u);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
      } else {
        // mark the references >= Ae of the boxes' cells.  Cells (cx, cy, *)
        // are consecutive in the list, so each (cx, cy) line of a box is one
        // run; runs are flattened over the lanes, 4 loads a lane at once.
        for (int t = w0 + lane; t < w1; t += 64) bm[t] = 0u;
        const int32_t* __restrict__ cs = cstart + (size_t)n * (KG_CELLS + 1);
        const int32_t* __restrict__ ls = list + (size_t)n * P2;
        const int nruns = runs_pre[4];
        int32_t* __restrict__ r_off = cl;      // run offsets (window area as scratch)
        int32_t* __restrict__ r_st = cl + 64;  // run starts in the list
        for (int r0 = 0; r0 < nruns; r0 += 64) {
          const int r = r0 + lane;
          const bool has = r < nruns;
          int g = 0;  // the row whose box holds run r
#pragma unroll
          for (int x = 1; x < 4; ++x) g += has && r >= runs_pre[x] ? 1 : 0;
          // (the shuffles read the row's lane 16g with every lane active)
          const int gx0 = __shfl(blo[0], 16 * g, 64), gy0 = __shfl(blo[1], 16 * g, 64);
          const int gz0 = __shfl(blo[2], 16 * g, 64), gz1 = __shfl(bhi[2], 16 * g, 64);
          const int gny = __shfl(ey, 16 * g, 64);
          int st = 0, ln = 0;
          if (has) {
            const int rl = r - runs_pre[g];
            const int base = ((gx0 + rl / gny) * KG_G + gy0 + rl % gny) * KG_G;
            st = cs[base + gz0];
            ln = cs[base + gz1 + 1] - st;
          }
          int incl = ln;
#pragma unroll
          for (int d = 1; d < 64; d <<= 1) {
            const int o = __shfl_up(incl, d, 64);
            if (lane >= d) incl += o;
          }
          const int tot = __shfl(incl, 63, 64);
          r_off[lane] = r < nruns ? incl - ln : 0x7fffffff;
          r_st[lane] = st;
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          for (int p0 = 0; p0 < tot; p0 += 256) {
            int jv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int pp = p0 + 64 * u + lane;
              jv[u] = -1;
              if (pp < tot) {
                int lo = 0;  // the last run starting at or before pp
#pragma unroll
                for (int step = 32; step >= 1; step >>= 1)
                  if (r_off[lo + step] <= pp) lo += step;
                jv[u] = ls[r_st[lo] + pp - r_off[lo]];
              }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
              if (jv[u] >= Ae) atomicOr(&bm[jv[u] >> 5], 1u << (jv[u] & 31));
          }
          __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
          __builtin_amdgcn_wave_barrier();
        }
      }
      {
        // windows of at most KG_WIN marked references in index order:
        // compact their indices, gather their coordinates into LDS (all
        // loads of a window in flight together), then run them as chunks
        int wcur = w0;
        while (wcur < w1) {
          const int wi = wcur + lane;
          uint32_t word = wi < w1 ? bm[wi] : 0u;
          const int pc = __builtin_popcount(word);
          int incl = pc;
#pragma unroll
          for (int d = 1; d < 64; d <<= 1) {
            const int o = __shfl_up(incl, d, 64);
            if (lane >= d) incl += o;
          }
          // the leading words whose marks fit (counts only grow with the lane)
          const uint64_t fit = __ballot(wi < w1 && incl <= KG_WIN);
          const int m = __builtin_popcountll(fit);  // >= 1: a word holds <= 32 marks
          const int total = __shfl(incl, m - 1, 64);
          __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
          __builtin_amdgcn_wave_barrier();  // the previous window's reads are done
          if (lane < m) {
            int o = incl - pc;
            while (word) {
              const int b = __builtin_ctz(word);
              word &= word - 1;
              cl[o++] = wi * 32 + b;
            }
          }
          wcur += m;
          __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
          __builtin_amdgcn_wave_barrier();
          if (total > 0) run(0, total, [&](int e) { return cl[e]; });
        }
      }
    }
  }
  if (!act) return;
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

struct KgLayout {
  int64_t hdr, cstart, list, total;
};
KgLayout kg_layout(int64_t N, int64_t P2) {
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  KgLayout L;
  L.hdr = 0;
  L.cstart = up(N * 8 * 4);
  L.list = L.cstart + up(N * (KG_CELLS + 1) * 4);
  L.total = L.list + up(N * P2 * 4);
  return L;
}

int kg_words(int64_t P2) { return (int)(((P2 + 31) / 32 + 63) / 64 * 64); }

template <int NORM, int KC, bool SORT>
void kg_launch(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2,
               const int32_t* order, const float* hdr, const int32_t* cs, const int32_t* ls,
               int N, int P1, int P2, int K, int A, int pad, int64_t* idxs, void* dists,
               hipStream_t s) {
  const int nqb = (P1 + 255) / 256;
  const int words = kg_words(P2);
  const size_t lds = (size_t)KG_WAVES * (words + KG_WIN + KNN_CHUNK * 64) * 4;
  hipLaunchKernelGGL((knn_grid_kernel<NORM, KC, SORT>), dim3(N * nqb), dim3(256), lds, s,
                     (const float*)p1, (const float*)p2, l1, l2, order, hdr, cs, ls, P1, P2, K, A,
                     nqb, words, pad, idxs, (float*)dists);
}

template <int NORM, bool SORT>
void kg_launch_k(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2,
                 const int32_t* order, const float* hdr, const int32_t* cs, const int32_t* ls,
                 int N, int P1, int P2, int K, int A, int pad, int64_t* idxs, void* dists,
                 hipStream_t s) {
  if (K <= 4) kg_launch<NORM, 4, SORT>(p1, p2, l1, l2, order, hdr, cs, ls, N, P1, P2, K, A, pad, idxs, dists, s);
  else if (K <= 8) kg_launch<NORM, 8, SORT>(p1, p2, l1, l2, order, hdr, cs, ls, N, P1, P2, K, A, pad, idxs, dists, s);
  else if (K <= 16) kg_launch<NORM, 16, SORT>(p1, p2, l1, l2, order, hdr, cs, ls, N, P1, P2, K, A, pad, idxs, dists, s);
  else kg_launch<NORM, 32, SORT>(p1, p2, l1, l2, order, hdr, cs, ls, N, P1, P2, K, A, pad, idxs, dists, s);
}

}  // namespace

// Reference prefix processed by brute force: about where the prefix costs
// as much as the box's references (both ~ sqrt(K * P2) per query).
constexpr int KG_PREFIX_MIN = 256, KG_PREFIX_MAX = 1024;
constexpr int64_t KG_MIN_P2 = 2048, KG_MAX_P2 = 32768;

bool knn_grid_applies(int dtype, int64_t D, int64_t K, int64_t P2) {
  return dtype == TPO_F32 && D == 3 && K >= 1 && K <= 32 && P2 >= KG_MIN_P2 && P2 <= KG_MAX_P2;
}

int64_t knn_grid_workspace(int64_t N, int64_t P2) { return kg_layout(N, P2).total; }

void launch_knn_grid(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2,
                     int32_t* order, int N, int P1, int P2, int K, int norm, int pad,
                     bool sort, int64_t* idxs, void* dists, void* ws, hipStream_t s) {
  const KgLayout L = kg_layout(N, P2);
  float* hdr = (float*)((char*)ws + L.hdr);
  int32_t* cs = (int32_t*)((char*)ws + L.cstart);
  int32_t* ls = (int32_t*)((char*)ws + L.list);
  hipLaunchKernelGGL(knn_grid_setup_kernel, dim3(2 * N), dim3(1024), 0, s, (const float*)p1, l1,
                     P1, order, (const float*)p2, l2, P2, N, hdr, cs, ls);
  int A = (int)std::sqrt(4.0 * K * (double)P2);
  A = std::max(KG_PREFIX_MIN, std::min(KG_PREFIX_MAX, A));
  A = std::max(A, K);
  if (norm == 1) {
    if (sort) kg_launch_k<1, true>(p1, p2, l1, l2, order, hdr, cs, ls, N, P1, P2, K, A, pad, idxs, dists, s);
    else kg_launch_k<1, false>(p1, p2, l1, l2, order, hdr, cs, ls, N, P1, P2, K, A, pad, idxs, dists, s);
  } else {
    if (sort) kg_launch_k<2, true>(p1, p2, l1, l2, order, hdr, cs, ls, N, P1, P2, K, A, pad, idxs, dists, s);
    else kg_launch_k<2, false>(p1, p2, l1, l2, order, hdr, cs, ls, N, P1, P2, K, A, pad, idxs, dists, s);
  }
}

}  // namespace tpo
