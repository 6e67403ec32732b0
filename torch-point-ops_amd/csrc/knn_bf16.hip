// knn_bf16.hip -- K nearest neighbours for bfloat16 points on the matrix
// cores (the high-D path; the reference's knn_cuda_forward, knn.cu:295-398,
// has no bfloat16 kernel and raises for it).
//
// Distances are squared L2 in float: d = |q|^2 + |r|^2 - 2 q.r, with the
// bfloat16 products exact in float, q.r summed by v_mfma_f32_32x32x16_bf16 and
// |q|^2, |r|^2 by a float FMA chain (knn_bf16_norms_kernel); d is clamped at 0.
// Each query's K nearest are returned sorted by (distance, index), distances
// rounded to bfloat16; rows past lengths1 and slots past lengths2 are (0, 0)
// as in the reference's version-2 layout.
//
// Layout of one v_mfma_f32_32x32x16_bf16 (checked on the device): lane l
// supplies 8 consecutive k of row/column l%32, k = 8(l/32)..8(l/32)+7, and
// receives column l%32, rows 8(v/4) + 4(l/32) + v%4 for v = 0..15.
//
// knn_bf16_slice_kernel: a workgroup of 4 waves owns 256 queries and one
// slice of the references; each wave multiplies two 32-query blocks (the
// MFMA columns) by every 32-reference tile of the slice, so each row
// fragment it loads feeds two MFMAs (operand traffic per FLOP halves against
// one block a wave).  A tile's fragments are loaded one tile ahead, with no
// synchronisation between waves.  v_permlane32_swap_b32 then exchanges the
// two accumulators' half-waves (checked on the device: swap(x, y) leaves
// x = [x_lo, y_lo], y = [x_hi, y_hi]), after which lane l holds all 32 rows of
// one query: block l/32, column l%32.  Each lane keeps its own sorted list of
// the KC best (KC >= K): candidates are queued per lane in LDS in increasing
// reference order and inserted in bulk by a branch-free network when some
// queue could overflow, so one pass serves every lane that has work;
// strict-less insertion keeps the lower index first among equal distances.
// Each lane writes the first K entries of its list for its slice, and
// knn_bf16_merge_kernel merges a query's slices.
#include <type_traits>

#include "knn_common.hpp"

#pragma clang fp contract(off)

namespace tpo {

typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));
typedef float f16v_t __attribute__((ext_vector_type(16)));

constexpr int KB_T = 32;                 // references per tile (MFMA rows)
constexpr int KB_WAVES = 4;
constexpr int KB_QW = 64 * KB_WAVES;     // queries per workgroup (two 32-query blocks a wave)
constexpr int KB_DMAX = 128;
constexpr int KB_QCAP = 16;              // queued candidates per lane
constexpr int KB_MAX_SLICES = 8;
constexpr int KB_NONE = 0x7fffffff;      // index of an empty list entry

__host__ __device__ inline int64_t kb_pad(int64_t n) { return (n + 31) & ~(int64_t)31; }

// out[r] = sum over d of p[r][d]^2 in float (rows of D bfloat16, D % 8 == 0)
__global__ __launch_bounds__(256) void knn_bf16_norms_kernel(const __bf16* __restrict__ p,
                                                             int64_t rows, int64_t stride_out,
                                                             int64_t rows_per_batch, int D,
                                                             float* __restrict__ out) {
  for (int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x; r < rows;
       r += (int64_t)gridDim.x * 256) {
    const bf8_t* x = reinterpret_cast<const bf8_t*>(p + r * D);
    float acc = 0.f;
    for (int d = 0; d < D / 8; ++d) {
      const bf8_t v = x[d];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = (float)v[e];
        acc = __builtin_fmaf(f, f, acc);
      }
    }
    const int64_t b = r / rows_per_batch;
    out[b * stride_out + (r - b * rows_per_batch)] = acc;
  }
}

// d[v] for a per-lane v in [0, 16): a 4-level select tree over registers
// (one ballot per level), so the array is never indexed dynamically
__device__ __forceinline__ float kb_sel16(const float (&d)[16], int v) {
  float a[8], b[4], e[2];
  const uint64_t m0 = __ballot(v & 1), m1 = __ballot(v & 2), m2 = __ballot(v & 4),
                 m3 = __ballot(v & 8);
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = csel(m0, d[2 * i], d[2 * i + 1]);
#pragma unroll
  for (int i = 0; i < 4; ++i) b[i] = csel(m1, a[2 * i], a[2 * i + 1]);
#pragma unroll
  for (int i = 0; i < 2; ++i) e[i] = csel(m2, b[2 * i], b[2 * i + 1]);
  return csel(m3, e[0], e[1]);
}

template <int KC>
__device__ __forceinline__ void kb_insert(float (&ld)[KC], int (&li)[KC], float d, int id) {
  // sorted insertion; a no-op when d is not below the last entry
  bool c[KC];
#pragma unroll
  for (int s = 0; s < KC; ++s) c[s] = d < ld[s];
#pragma unroll
  for (int s = KC - 1; s > 0; --s) {
    ld[s] = c[s - 1] ? ld[s - 1] : (c[s] ? d : ld[s]);
    li[s] = c[s - 1] ? li[s - 1] : (c[s] ? id : li[s]);
  }
  ld[0] = c[0] ? d : ld[0];
  li[0] = c[0] ? id : li[0];
}

// Work split: query blocks of 256 and reference slices (one workgroup each).
struct KbPlan {
  int nqb, slices;
};
static KbPlan kb_plan(int64_t N, int64_t P1, int64_t P2) {
  KbPlan p;
  p.nqb = (int)((P1 + KB_QW - 1) / KB_QW);
  const int64_t wgs = N * (int64_t)p.nqb;
  int64_t s = wgs > 0 ? (512 + wgs - 1) / wgs : 1;  // about two workgroups per CU
  const int64_t tiles = (P2 + KB_T - 1) / KB_T;
  s = std::min<int64_t>(s, std::max<int64_t>(1, tiles / 16));  // at least 16 tiles a slice
  p.slices = (int)std::max<int64_t>(1, std::min<int64_t>(s, KB_MAX_SLICES));
  return p;
}

// KS k-steps of 16 dims; HALF: D % 16 == 8, so the upper half of the last
// step lies past D (its operands are zero)
template <int KS, bool HALF, int KC>
__global__ __launch_bounds__(256) void knn_bf16_slice_kernel(
    const __bf16* __restrict__ p1, const __bf16* __restrict__ p2, const int64_t* __restrict__ len1,
    const int64_t* __restrict__ len2, int P1, int P2, int D, int K, int nqb, int slices,
    const float* __restrict__ qn, const float* __restrict__ rn, int2* __restrict__ part) {
  __shared__ float s_qd[KB_WAVES][KB_QCAP][64];
  __shared__ int s_qi[KB_WAVES][KB_QCAP][64];

  // logical block = ((n * slices) + slice) * nqb + query block: the blocks
  // reading one slice are consecutive, hence on one XCD
  const int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int qb = lb % nqb, ns = lb / nqb;
  const int sl = ns % slices, n = ns / slices;
  int64_t l1 = len1[n], l2 = len2[n];
  l1 = l1 < 0 ? 0 : (l1 > P1 ? P1 : l1);
  l2 = l2 < 0 ? 0 : (l2 > P2 ? P2 : l2);
  const int L2 = (int)l2;
  const int tid = threadIdx.x, w = wave_id(), lane = lane_id(), j = lane & 31, h = lane >> 5;
  const int qw = qb * KB_QW + 64 * w;  // the wave's blocks: queries qw + 32 b + column
  const int q = qw + lane;             // this lane's query after the swap: block h, column j

  // column operands of both blocks: query qw + 32 b + j, dims 16s + 8h .. + 7
  // (zero past D)
  bf8_t bq0[KS], bq1[KS];
  {
    const __bf16* __restrict__ qp0 = p1 + ((size_t)n * P1 + min(qw + j, P1 - 1)) * D;
    const __bf16* __restrict__ qp1 = p1 + ((size_t)n * P1 + min(qw + 32 + j, P1 - 1)) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int d0 = 16 * s + 8 * h;
      bq0[s] = d0 < D ? *reinterpret_cast<const bf8_t*>(qp0 + d0) : bf8_t{};
      bq1[s] = d0 < D ? *reinterpret_cast<const bf8_t*>(qp1 + d0) : bf8_t{};
    }
  }
  const float qq = qn[(size_t)n * kb_pad(P1) + min(q, P1 - 1)];
  const __bf16* __restrict__ rb = p2 + (size_t)n * P2 * D;
  const float* __restrict__ rr = rn + (size_t)n * kb_pad(P2);

  // the slice's tiles
  const int ntiles = (L2 + KB_T - 1) / KB_T;
  const int tps = (ntiles + slices - 1) / slices;
  const int t0 = min(sl * tps, ntiles), t1 = min(ntiles, t0 + tps);

  float ld[KC];
  int li[KC];
#pragma unroll
  for (int s = 0; s < KC; ++s) {
    ld[s] = Lim<float>::inf();
    li[s] = KB_NONE;
  }
  int nq_ = 0;  // queued candidates of this lane
  // insert the queue in order: each pass a lane first skips (cheaply) the
  // entries no longer below its list's last one, then inserts its next entry,
  // so the passes number the largest count of useful insertions in the wave
  auto drain = [&]() {
    int k = 0;
    for (;;) {
      while (k < nq_ && !(s_qd[w][k][lane] < ld[KC - 1])) ++k;
      if (__ballot(k < nq_) == 0) break;
      if (k < nq_) {
        kb_insert<KC>(ld, li, s_qd[w][k][lane], s_qi[w][k][lane]);
        ++k;
      }
    }
    nq_ = 0;
  };

  // Row operand of tile t for this lane: reference base + j, dims 16s + 8h
  // .. + 7, and the norms of the lane's rows.  Loads are unconditional (row
  // clamped into [0, L2), a half past D re-reads the step's lower half and is
  // zeroed at use), so they issue together, one tile ahead.
  bf8_t an[KS];
  float4 rn4[8];  // norms of rows 4i .. 4i + 3
  auto load_rows = [&](int t) {
    const int tc = min(t, ntiles - 1), base = tc * KB_T;  // a tile past the slice re-reads the last
    const __bf16* __restrict__ ra = rb + (size_t)min(base + j, L2 - 1) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int d0 = (HALF && s == KS - 1) ? 16 * s : 16 * s + 8 * h;
      an[s] = *reinterpret_cast<const bf8_t*>(ra + d0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) rn4[i] = *reinterpret_cast<const float4*>(rr + base + 4 * i);
  };
  if (t0 < t1) load_rows(t0);
  for (int t = t0; t < t1; ++t) {
    const int base = t * KB_T;
    bf8_t a[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) a[s] = an[s];
    if constexpr (HALF) a[KS - 1] = h ? bf8_t{} : a[KS - 1];
    float4 r4[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) r4[i] = rn4[i];
    load_rows(t + 1);  // the next tile's loads are in flight during this one
    f16v_t acc0 = {}, acc1 = {};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s], bq0[s], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s], bq1[s], acc1, 0, 0, 0);
    }
    // lane l: block l/32, column l%32; rows 8(v/4) + v%4 in acc0[v], rows
    // 8(v/4) + 4 + v%4 in acc1[v]
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc0[v]), __float_as_uint(acc1[v]), false, false);
      acc0[v] = __uint_as_float(r[0]);
      acc1[v] = __uint_as_float(r[1]);
    }
    // Two halves of 16 rows (8-row groups 2c, 2c + 1), in increasing row
    // order.  The filter compares the unclamped value (a negative one passes
    // it, and the pushed value is clamped at 0); only the last tile can hold
    // rows past L2.
    const bool partial = base + KB_T > L2;
    {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const float thr = ld[KC - 1];
        float dv[16];
        uint32_t m = 0;  // bit v: row 16c + v is below the list's end
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
          const int g = 2 * c + gg;
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const float4 rq = r4[2 * g + hh];  // rows 8g + 4hh ..
            const float rv[4] = {rq.x, rq.y, rq.z, rq.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float a = hh ? acc1[4 * g + e] : acc0[4 * g + e];
              float d = __builtin_fmaf(-2.f, a, qq + rv[e]);
              if (partial) d = base + 8 * g + 4 * hh + e < L2 ? d : Lim<float>::inf();
              const int v = 8 * gg + 4 * hh + e;  // row 16c + v
              dv[v] = d;
              m |= (d < thr ? 1u : 0u) << v;
            }
          }
        }
        if (__ballot(m != 0) != 0) {  // some lane has a candidate in these rows
          if (__ballot(nq_ + __builtin_popcount(m) > KB_QCAP) != 0) drain();  // queues within capacity
          // only the set bits: the wave pays max-over-lanes(candidates), not 16
          // rows of branches (thr may predate a drain: a stale entry inserts
          // as a no-op)
          while (m) {
            const int v = __builtin_ctz(m);
            m &= m - 1;
            s_qd[w][nq_][lane] = fmaxf(kb_sel16(dv, v), 0.f);
            s_qi[w][nq_][lane] = base + 16 * c + v;
            ++nq_;
          }
        }
      }
    }
  }
  drain();

  // the first K entries of this lane's list
  if (q < P1 && q < l1) {
    int2* __restrict__ out = part + (((size_t)n * P1 + q) * slices + sl) * K;
#pragma unroll
    for (int s = 0; s < KC; ++s)
      if (s < K) out[s] = make_int2(__float_as_int(ld[s]), li[s]);
  }
}

// One thread per query row: merge its nl sorted lists of K, smallest
// (distance, index) first; rows past lengths1 and empty slots are (0, 0).
template <int MAXL>
__global__ __launch_bounds__(256) void knn_bf16_merge_kernel(const int2* __restrict__ part,
                                                             const int64_t* __restrict__ len1,
                                                             int64_t rows, int P1, int K, int nl,
                                                             int64_t* __restrict__ idxs,
                                                             __bf16* __restrict__ dists) {
  const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (row >= rows) return;
  const int64_t n = row / P1;
  const int q = (int)(row - n * P1);
  int64_t l1 = len1[n];
  l1 = l1 < 0 ? 0 : (l1 > P1 ? P1 : l1);
  int64_t* __restrict__ io = idxs + row * K;
  __bf16* __restrict__ dout = dists + row * K;
  if (q >= l1) {
    for (int k = 0; k < K; ++k) {
      io[k] = 0;
      dout[k] = (__bf16)0.f;
    }
    return;
  }
  const int2* __restrict__ lists = part + row * (int64_t)nl * K;
  int ptr[MAXL];
  float hd[MAXL];
  int hi[MAXL];
#pragma unroll
  for (int L = 0; L < MAXL; ++L) {
    ptr[L] = 0;
    const int2 e = L < nl ? lists[(size_t)L * K] : make_int2(__float_as_int(Lim<float>::inf()), KB_NONE);
    hd[L] = __int_as_float(e.x);
    hi[L] = e.y;
  }
  for (int k = 0; k < K; ++k) {
    float bd = hd[0];
    int bi = hi[0], bl = 0;
#pragma unroll
    for (int L = 1; L < MAXL; ++L) {
      if (hd[L] < bd || (hd[L] == bd && hi[L] < bi)) {
        bd = hd[L];
        bi = hi[L];
        bl = L;
      }
    }
    const bool real = bi != KB_NONE;  // fewer than K references
    io[k] = real ? (int64_t)bi : 0;
    dout[k] = real ? (__bf16)bd : (__bf16)0.f;
#pragma unroll
    for (int L = 0; L < MAXL; ++L) {
      if (L == bl) {
        const int p = ++ptr[L];
        const int2 e = p < K ? lists[(size_t)L * K + p] : make_int2(__float_as_int(Lim<float>::inf()), KB_NONE);
        hd[L] = __int_as_float(e.x);
        hi[L] = e.y;
      }
    }
  }
}

static int64_t kb_align(int64_t x) { return (x + 255) / 256 * 256; }

// norms (float per point, rows padded to 32), then the partial lists
int64_t knn_bf16_workspace(int64_t N, int64_t P1, int64_t P2, int64_t K) {
  const KbPlan p = kb_plan(N, P1, P2);
  return kb_align(N * (kb_pad(P1) + kb_pad(P2)) * 4) + kb_align(N * P1 * p.slices * K * 8);
}

bool knn_bf16_supported(int64_t D, int64_t K, int norm) {
  return norm == 2 && D % 8 == 0 && D >= 8 && D <= KB_DMAX && K >= 1 && K <= 32;
}

template <int KS, bool HALF, int KC>
static void kb_launch(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2,
                      int N, int P1, int P2, int D, int K, const float* qn, const float* rn,
                      int2* part, hipStream_t s) {
  const KbPlan p = kb_plan(N, P1, P2);
  hipLaunchKernelGGL((knn_bf16_slice_kernel<KS, HALF, KC>), dim3(N * p.nqb * p.slices), dim3(256), 0, s,
                     (const __bf16*)p1, (const __bf16*)p2, l1, l2, P1, P2, D, K, p.nqb, p.slices,
                     qn, rn, part);
}

template <int KC>
static void kb_dispatch_ks(int D, const void* p1, const void* p2, const int64_t* l1,
                           const int64_t* l2, int N, int P1, int P2, int K, const float* qn,
                           const float* rn, int2* part, hipStream_t s) {
  // D % 8 == 0, 8 <= D <= 128: D / 8 = 2 KS - HALF
#define KB_CASE(DD, KS_, HALF_) \
  case DD: kb_launch<KS_, HALF_, KC>(p1, p2, l1, l2, N, P1, P2, D, K, qn, rn, part, s); break;
  switch (D) {
    KB_CASE(8, 1, true) KB_CASE(16, 1, false) KB_CASE(24, 2, true) KB_CASE(32, 2, false)
    KB_CASE(40, 3, true) KB_CASE(48, 3, false) KB_CASE(56, 4, true) KB_CASE(64, 4, false)
    KB_CASE(72, 5, true) KB_CASE(80, 5, false) KB_CASE(88, 6, true) KB_CASE(96, 6, false)
    KB_CASE(104, 7, true) KB_CASE(112, 7, false) KB_CASE(120, 8, true)
    default: kb_launch<8, false, KC>(p1, p2, l1, l2, N, P1, P2, D, K, qn, rn, part, s); break;
  }
#undef KB_CASE
}

void launch_knn_bf16(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2, int N,
                     int P1, int P2, int D, int K, int64_t* idxs, void* dists, void* ws,
                     hipStream_t s) {
  const KbPlan p = kb_plan(N, P1, P2);
  float* qn = reinterpret_cast<float*>(ws);
  float* rn = qn + (size_t)N * kb_pad(P1);
  int2* part = reinterpret_cast<int2*>(reinterpret_cast<char*>(ws) +
                                       kb_align((int64_t)N * (kb_pad(P1) + kb_pad(P2)) * 4));
  const int64_t r1 = (int64_t)N * P1, r2 = (int64_t)N * P2;
  if (r1 > 0)
    hipLaunchKernelGGL(knn_bf16_norms_kernel, dim3((unsigned)std::min<int64_t>((r1 + 255) / 256, 65536)),
                       dim3(256), 0, s, (const __bf16*)p1, r1, kb_pad(P1), (int64_t)P1, D, qn);
  if (r2 > 0)
    hipLaunchKernelGGL(knn_bf16_norms_kernel, dim3((unsigned)std::min<int64_t>((r2 + 255) / 256, 65536)),
                       dim3(256), 0, s, (const __bf16*)p2, r2, kb_pad(P2), (int64_t)P2, D, rn);
  if (r1 == 0) return;
  if (K <= 16) kb_dispatch_ks<16>(D, p1, p2, l1, l2, N, P1, P2, K, qn, rn, part, s);
  else kb_dispatch_ks<32>(D, p1, p2, l1, l2, N, P1, P2, K, qn, rn, part, s);
  const int nl = p.slices;
  const dim3 mg((unsigned)((r1 + 255) / 256)), mb(256);
  if (nl <= 4)
    hipLaunchKernelGGL(knn_bf16_merge_kernel<4>, mg, mb, 0, s, (const int2*)part, l1, r1, P1, K, nl, idxs, (__bf16*)dists);
  else if (nl <= 8)
    hipLaunchKernelGGL(knn_bf16_merge_kernel<8>, mg, mb, 0, s, (const int2*)part, l1, r1, P1, K, nl, idxs, (__bf16*)dists);
  else
    hipLaunchKernelGGL(knn_bf16_merge_kernel<KB_MAX_SLICES>, mg, mb, 0, s, (const int2*)part, l1, r1, P1, K, nl, idxs, (__bf16*)dists);
}

}  // namespace tpo
