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
// receives column l%32, rows 8(v/4) + 4(l/32) + v%4 for v = 0..15.  Queries
// are the 32 columns of a workgroup, references the rows of 32-point tiles;
// the workgroup's 4 waves take every 4th tile.  Each lane thus sees 16
// references per tile for its query and keeps its own sorted list of the KC
// best (KC >= K): a candidate below the list's last entry is inserted by a
// branch-free network.  References reach a lane in increasing index order, so
// strict-less insertion keeps the lower index first among equal distances.
// Candidates are first queued per lane in LDS (in index order) and inserted
// in bulk when some lane's queue is about to overflow, so one pass of the
// insertion network serves every lane that has work.  At the end the 8 lists
// of a query (2 lanes x 4 waves) are merged in LDS.
#include "tpo_common.hpp"

#pragma clang fp contract(off)

namespace tpo {

typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));
typedef float f16v_t __attribute__((ext_vector_type(16)));

constexpr int KB_Q = 32;  // queries per workgroup (MFMA columns)
constexpr int KB_T = 32;  // references per tile (MFMA rows)
constexpr int KB_WAVES = 4;

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

constexpr int KB_QCAP = 16;  // queued candidates per lane

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

// KS k-steps of 16 dims; HALF: D % 16 == 8, so the upper half of the last
// step lies past D (its operands are zero)
template <int KS, bool HALF, int KC>
__global__ __launch_bounds__(256) void knn_bf16_kernel(
    const __bf16* __restrict__ p1, const __bf16* __restrict__ p2, const int64_t* __restrict__ len1,
    const int64_t* __restrict__ len2, int P1, int P2, int D, int K, int nqb,
    const float* __restrict__ qn, const float* __restrict__ rn, int64_t* __restrict__ idxs,
    __bf16* __restrict__ dists) {
  // per-lane candidate queues during the scan, the 8 lists of each query after
  struct Queues {
    float d[KB_WAVES][KB_QCAP][64];
    int i[KB_WAVES][KB_QCAP][64];
  };
  struct Lists {
    float d[KB_Q][2 * KB_WAVES][KC];
    int i[KB_Q][2 * KB_WAVES][KC];
  };
  __shared__ union {
    Queues q;
    Lists l;
  } sm;
  // s_bound[w][j]: wave w's bound for query j (see below)
  __shared__ float s_bound[KB_WAVES][KB_Q];

  const int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int n = lb / nqb, qb = lb - n * nqb;
  int64_t l1 = len1[n], l2 = len2[n];
  l1 = l1 < 0 ? 0 : (l1 > P1 ? P1 : l1);
  l2 = l2 < 0 ? 0 : (l2 > P2 ? P2 : l2);
  const int L2 = (int)l2;
  const int w = wave_id(), lane = lane_id(), j = lane & 31, h = lane >> 5;
  const int q = qb * KB_Q + j;
  const int qc = min(q, P1 - 1);

  // column operand: query qc, dims 16s + 8h .. 16s + 8h + 7 (zero past D)
  const __bf16* __restrict__ qp = p1 + ((size_t)n * P1 + qc) * D;
  bf8_t bq[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int d0 = 16 * s + 8 * h;
    bq[s] = d0 < D ? *reinterpret_cast<const bf8_t*>(qp + d0) : bf8_t{};
  }
  const float qq = qn[(size_t)n * kb_pad(P1) + qc];
  const __bf16* __restrict__ rb = p2 + (size_t)n * P2 * D;
  const float* __restrict__ rr = rn + (size_t)n * kb_pad(P2);

  float ld[KC];
  int li[KC];
#pragma unroll
  for (int s = 0; s < KC; ++s) {
    ld[s] = Lim<float>::inf();
    li[s] = 0x7fffffff;
  }
  // Shared bound.  The 8 lists of a query (2 lanes x 4 waves) hold disjoint
  // references, so if each has at least c = ceil(K / 8) entries, 8c >= K of
  // them are <= the largest of the 8 lists' c-th entries: that value bounds
  // the query's K-th distance, and a candidate above it can never be among
  // the K nearest.  One strictly above is dropped; equality is kept so that
  // the (distance, index) order of ties is unaffected.  Lists only improve,
  // so an older published value is still a valid bound.
  if (lane < KB_Q) s_bound[w][lane] = Lim<float>::inf();
  __syncthreads();
  const int cth = (K + 7) / 8 - 1;  // 0..3
  float sb = Lim<float>::inf();
  auto refresh_bound = [&]() {
    const float own = cth == 0 ? ld[0] : (cth == 1 ? ld[1] : (cth == 2 ? ld[2] : ld[3]));
    const float pair = fmaxf(own, __shfl_xor(own, 32));
    if (h == 0) __hip_atomic_store(&s_bound[w][j], pair, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    float b = pair;
#pragma unroll
    for (int v = 0; v < KB_WAVES; ++v)
      if (v != w) b = fmaxf(b, __hip_atomic_load(&s_bound[v][j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
    sb = b;
  };
  int nq_ = 0;  // queued candidates of this lane
  // insert the queue in order: each pass a lane first skips (cheaply) the
  // entries no longer below its list's last one, then inserts its next entry,
  // so the passes number the largest count of useful insertions in the wave
  auto drain = [&]() {
    int k = 0;
    for (;;) {
      while (k < nq_ && !(sm.q.d[w][k][lane] < ld[KC - 1])) ++k;
      if (__ballot(k < nq_) == 0) break;
      if (k < nq_) {
        kb_insert<KC>(ld, li, sm.q.d[w][k][lane], sm.q.i[w][k][lane]);
        ++k;
      }
    }
    nq_ = 0;
  };

  const int ntiles = (L2 + KB_T - 1) / KB_T;
  // Row operand of tile t for this lane: reference base + j, dims 16s + 8h ..
  // + 7.  Loads are unconditional (row clamped into [0, L2), a half past D
  // re-reads the step's lower half and is zeroed at use), so they all issue
  // together; each tile's loads are made one tile ahead.
  bf8_t an[KS];
  auto load_rows = [&](int t) {
    const int r = min(t * KB_T + j, L2 - 1);
    const __bf16* __restrict__ ra = rb + (size_t)max(r, 0) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int d0 = (HALF && s == KS - 1) ? 16 * s : 16 * s + 8 * h;
      an[s] = *reinterpret_cast<const bf8_t*>(ra + d0);
    }
  };
  if (w < ntiles) load_rows(w);
  for (int t = w; t < ntiles; t += KB_WAVES) {
    const int base = t * KB_T;
    bf8_t a[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) a[s] = an[s];
    if constexpr (HALF) a[KS - 1] = h ? bf8_t{} : a[KS - 1];
    load_rows(t + KB_WAVES);  // the wave's next tile, in flight during this one
    f16v_t acc = {};
#pragma unroll
    for (int s = 0; s < KS; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s], bq[s], acc, 0, 0, 0);
    if ((t & (4 * KB_WAVES - 1)) == w) refresh_bound();  // every 4th tile of the wave
    float dv[16];
    int pc = 0;
    // below the own list's last entry and not above the shared bound
    const float thr = fminf(ld[KC - 1], sb < Lim<float>::inf() ? __uint_as_float(__float_as_uint(sb) + 1u) : sb);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 r4 = *reinterpret_cast<const float4*>(rr + base + 8 * g + 4 * h);
      const float rv[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int v = 4 * g + e;
        const int i = 8 * g + 4 * h + e;
        float d = fmaxf(__builtin_fmaf(-2.f, acc[v], qq + rv[e]), 0.f);
        d = base + i < L2 ? d : Lim<float>::inf();
        dv[v] = d;
        pc += d < thr ? 1 : 0;
      }
    }
    if (__ballot(nq_ + pc > KB_QCAP) != 0) drain();  // keep every queue within capacity
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      if (dv[v] < thr) {  // thr may predate a drain: a stale entry inserts as a no-op
        sm.q.d[w][nq_][lane] = dv[v];
        sm.q.i[w][nq_][lane] = base + 8 * (v >> 2) + 4 * h + (v & 3);
        ++nq_;
      }
    }
  }
  drain();
  __syncthreads();  // the queues' LDS becomes the lists'
#pragma unroll
  for (int s = 0; s < KC; ++s) {
    sm.l.d[j][2 * w + h][s] = ld[s];
    sm.l.i[j][2 * w + h][s] = li[s];
  }
  __syncthreads();

  // merge the 8 sorted lists of query j (threads 0..31), smallest (d, index) first
  if (threadIdx.x < KB_Q && q < P1) {
    const size_t row = (size_t)n * P1 + q;
    int64_t* __restrict__ io = idxs + row * K;
    __bf16* __restrict__ dout = dists + row * K;
    if (q >= l1) {
      for (int k = 0; k < K; ++k) {
        io[k] = 0;
        dout[k] = (__bf16)0.f;
      }
    } else {
      int ptr[2 * KB_WAVES] = {};
      for (int k = 0; k < K; ++k) {
        float bd = Lim<float>::inf();
        int bi = 0x7fffffff, bl = 0;
#pragma unroll
        for (int L = 0; L < 2 * KB_WAVES; ++L) {
          const int p = ptr[L];
          const float d = p < KC ? sm.l.d[j][L][p] : Lim<float>::inf();
          const int i = p < KC ? sm.l.i[j][L][p] : 0x7fffffff;
          if (d < bd || (d == bd && i < bi)) {
            bd = d;
            bi = i;
            bl = L;
          }
        }
#pragma unroll
        for (int L = 0; L < 2 * KB_WAVES; ++L) ptr[L] += L == bl ? 1 : 0;
        const bool real = bi != 0x7fffffff;  // fewer than K references
        io[k] = real ? (int64_t)bi : 0;
        dout[k] = real ? (__bf16)bd : (__bf16)0.f;
      }
    }
  }
}

int64_t knn_bf16_workspace(int64_t N, int64_t P1, int64_t P2) {
  return ((N * (kb_pad(P1) + kb_pad(P2)) * 4 + 255) / 256) * 256;
}

bool knn_bf16_supported(int64_t D, int64_t K, int norm) {
  return norm == 2 && D % 8 == 0 && D >= 8 && D <= 128 && K >= 1 && K <= 32;
}

template <int KS, bool HALF, int KC>
static void kb_launch(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2,
                      int N, int P1, int P2, int D, int K, const float* qn, const float* rn,
                      int64_t* idxs, void* dists, hipStream_t s) {
  const int nqb = (P1 + KB_Q - 1) / KB_Q;
  hipLaunchKernelGGL((knn_bf16_kernel<KS, HALF, KC>), dim3(N * nqb), dim3(256), 0, s,
                     (const __bf16*)p1, (const __bf16*)p2, l1, l2, P1, P2, D, K, nqb, qn, rn, idxs,
                     (__bf16*)dists);
}

template <int KC>
static void kb_dispatch_ks(int D, const void* p1, const void* p2, const int64_t* l1,
                           const int64_t* l2, int N, int P1, int P2, int K, const float* qn,
                           const float* rn, int64_t* idxs, void* dists, hipStream_t s) {
  // D % 8 == 0, 8 <= D <= 128: D / 8 = 2 KS - HALF
#define KB_CASE(DD, KS_, HALF_) \
  case DD: kb_launch<KS_, HALF_, KC>(p1, p2, l1, l2, N, P1, P2, D, K, qn, rn, idxs, dists, s); break;
  switch (D) {
    KB_CASE(8, 1, true) KB_CASE(16, 1, false) KB_CASE(24, 2, true) KB_CASE(32, 2, false)
    KB_CASE(40, 3, true) KB_CASE(48, 3, false) KB_CASE(56, 4, true) KB_CASE(64, 4, false)
    KB_CASE(72, 5, true) KB_CASE(80, 5, false) KB_CASE(88, 6, true) KB_CASE(96, 6, false)
    KB_CASE(104, 7, true) KB_CASE(112, 7, false) KB_CASE(120, 8, true)
    default: kb_launch<8, false, KC>(p1, p2, l1, l2, N, P1, P2, D, K, qn, rn, idxs, dists, s); break;
  }
#undef KB_CASE
}

void launch_knn_bf16(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2, int N,
                     int P1, int P2, int D, int K, int64_t* idxs, void* dists, void* ws,
                     hipStream_t s) {
  float* qn = reinterpret_cast<float*>(ws);
  float* rn = qn + (size_t)N * kb_pad(P1);
  const int64_t r1 = (int64_t)N * P1, r2 = (int64_t)N * P2;
  if (r1 > 0)
    hipLaunchKernelGGL(knn_bf16_norms_kernel, dim3((unsigned)std::min<int64_t>((r1 + 255) / 256, 65536)),
                       dim3(256), 0, s, (const __bf16*)p1, r1, kb_pad(P1), (int64_t)P1, D, qn);
  if (r2 > 0)
    hipLaunchKernelGGL(knn_bf16_norms_kernel, dim3((unsigned)std::min<int64_t>((r2 + 255) / 256, 65536)),
                       dim3(256), 0, s, (const __bf16*)p2, r2, kb_pad(P2), (int64_t)P2, D, rn);
  if (K <= 16) kb_dispatch_ks<16>(D, p1, p2, l1, l2, N, P1, P2, K, qn, rn, idxs, dists, s);
  else kb_dispatch_ks<32>(D, p1, p2, l1, l2, N, P1, P2, K, qn, rn, idxs, dists, s);
}

}  // namespace tpo
