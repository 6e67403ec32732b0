// knn_bf16.hip -- K nearest neighbours for bfloat16 points on the matrix
// cores (the high-D path; the reference's knn_cuda_forward, knn.cu:295-398,
// has no bfloat16 kernel and raises for it).
//
// Distances are squared L2 in float: d = |q|^2 + |r|^2 - 2 q.r, summed as one
// v_mfma_f32_32x32x16_bf16 chain: the query operand is -2 q (exact in
// bfloat16; the products are exact in float), and one more k-step adds |q|^2
// and |r|^2 (float, each from an FMA chain over the point's bfloat16 values,
// knn_bf16_norms_kernel) as three bfloat16 pieces each, whose sum is the float
// exactly (for norms above ~1e-33); d is clamped at 0.
// Each query's K nearest are returned sorted by (distance, index), distances
// rounded to bfloat16; rows past lengths1 and slots past lengths2 are (0, 0)
// as in the reference's version-2 layout.
//
// Layout of one v_mfma_f32_32x32x16_bf16 (checked on the device): lane l
// supplies 8 consecutive k of row/column l%32, k = 8(l/32)..8(l/32)+7, and
// receives column l%32, rows 8(v/4) + 4(l/32) + v%4 for v = 0..15.
//
// Two passes share that arithmetic.  In both, a workgroup of 4 waves owns
// 256 queries and one slice of the references, and each wave multiplies two
// 32-query blocks (the MFMA columns) by every 32-reference tile of the slice,
// staged once per workgroup in LDS, so each row fragment feeds two MFMAs.
//
// Candidate pass (clouds of at least max(4096, 1536 K) references):
// knn_bf16_tau_kernel first bounds each query by the 8th smallest of its
// minimum distances over 64 sampled tiles; knn_bf16_cand_kernel stores every
// distance at or below the bound as a 64-bit (distance, index) key in a
// region per (query, slice), and knn_bf16_cmerge_kernel selects each row's K
// from its candidates (a distance histogram, then ranks among the few that
// can be in the K).  Rows whose regions overflowed or that hold fewer than K
// candidates are listed for the exact pass.
//
// Exact pass (smaller clouds, and the listed rows): knn_bf16_slice_kernel.
// v_permlane32_swap_b32 exchanges the two accumulators' half-waves (checked
// on the device: swap(x, y) leaves x = [x_lo, y_lo], y = [x_hi, y_hi]), after
// which lane l holds all 32 rows of one query: block l/32, column l%32.  Each
// lane keeps its own sorted list of the KC best (KC >= K) keys: candidates
// are queued per lane in LDS and, when some queue could overflow, merged in
// groups of 8 by a sorting network and a bitonic merge in registers, so one
// branch-free pass serves every lane of the wave.  Each lane writes the first
// K entries of its list for its slice, and knn_bf16_merge_kernel merges a
// query's slices.  The key order puts the lower index first among equal
// distances in both passes.
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
// The sampled bound: the KB_TK-th smallest of each query's minimum distances
// over KB_TS reference tiles spread over its cloud (KB_TP workgroups of query
// blocks, KB_TS / KB_TP tiles each); see kb_sampled for the clouds that take
// one (the others' bound is +inf: every row then overflows or falls short and
// takes the exact pass).
constexpr int KB_TS = 64;
constexpr int KB_TP = 8;
constexpr int KB_TK = 8;
// The sampled bound applies to clouds of at least 2 KB_TS tiles and 1536 K
// references: about one reference in 260 lies at or below it (the 8th of 64
// tile minima), so a row then has ~6 K candidates on average; with fewer,
// rows left short (and rerun) would be common.
__host__ __device__ inline bool kb_sampled(int64_t L2, int64_t K) {
  return (L2 + KB_T - 1) / KB_T >= 2 * KB_TS && L2 >= 1536 * K;
}
// Under the bound: candidate slots per (query, slice), shared by the two
// half-waves that hold the query's rows (one fills up from slot 0, the other
// down from the last; a multiple of 64), and at most KB_CMAX_SLICES slices
constexpr int KB_CAP = 128;
constexpr int KB_CMAX_SLICES = 16;

__host__ __device__ inline int64_t kb_pad(int64_t n) { return (n + 31) & ~(int64_t)31; }

// out[r] = sum over d of p[r][d]^2 in float (rows of D bfloat16, D % 8 == 0,
// D <= 128): 16 lanes a row, lane c summing dims 8c .. 8c + 7 by an FMA chain
// from one 16-byte load, then the 16 partial sums added pairwise in a fixed
// order (lanes 8 apart, then 4, 2, 1).  One launch for both clouds: the
// first nb1 blocks take p1's rows (padded to 32 a batch in the output), the
// rest p2's.
__global__ __launch_bounds__(256) void knn_bf16_norms_kernel(
    const __bf16* __restrict__ p1, int64_t rows1, int64_t per1, float* __restrict__ out1,
    const __bf16* __restrict__ p2, int64_t rows2, int64_t per2, float* __restrict__ out2, int D,
    int64_t nb1) {
  const bool second = blockIdx.x >= nb1;  // block-uniform
  const __bf16* __restrict__ p = second ? p2 : p1;
  const int64_t rows = second ? rows2 : rows1, per = second ? per2 : per1;
  float* __restrict__ out = second ? out2 : out1;
  const int c = threadIdx.x & 15;
  const int64_t r = ((int64_t)(blockIdx.x - (second ? nb1 : 0)) * 256 + threadIdx.x) >> 4;
  const bool live = r < rows;
  float acc = 0.f;
  if (live && 8 * c < D) {
    const bf8_t v = *reinterpret_cast<const bf8_t*>(p + r * D + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = (float)v[e];
      acc = __builtin_fmaf(f, f, acc);
    }
  }
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  if (live && c == 0) {
    const int64_t b = r / per;
    out[b * kb_pad(per) + (r - b * per)] = acc;
  }
}

// d[v] for a per-lane v in [0, 16): a 4-level select tree over registers
// (a lane mask per level), so the array is never indexed dynamically
__device__ __forceinline__ float kb_sel16(const float (&d)[16], int v) {
  float a[8], b[4], e[2];
  const uint32_t m0 = bit_mask(v, 0), m1 = bit_mask(v, 1), m2 = bit_mask(v, 2),
                 m3 = bit_mask(v, 3);
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = csel(m0, d[2 * i], d[2 * i + 1]);
#pragma unroll
  for (int i = 0; i < 4; ++i) b[i] = csel(m1, a[2 * i], a[2 * i + 1]);
#pragma unroll
  for (int i = 0; i < 2; ++i) e[i] = csel(m2, b[2 * i], b[2 * i + 1]);
  return csel(m3, e[0], e[1]);
}

// The norm operand of the extra k-step: [h, m, l, 1, 1, 1, 0, 0] for a
// reference row, [1, 1, 1, h, m, l, 0, 0] for a query column, with
// h + m + l = x: x rounded to bfloat16, the (exact) remainder rounded, and the
// rest, itself exact in bfloat16 unless it is denormal (|x| below ~1e-33: an
// absolute error under 1e-38).  x = +inf gives NaN pieces.
__device__ __forceinline__ bf8_t kb_norm_operand(float x, bool row) {
  const __bf16 hi = (__bf16)x;
  const float r = x - (float)hi;
  const __bf16 mi = (__bf16)r;
  const __bf16 lo = (__bf16)(r - (float)mi);
  const __bf16 one = (__bf16)1.f, z = (__bf16)0.f;
  return row ? bf8_t{hi, mi, lo, one, one, one, z, z} : bf8_t{one, one, one, hi, mi, lo, z, z};
}

// -2 v elementwise (exact in bfloat16 below the overflow range)
__device__ __forceinline__ bf8_t kb_neg2(bf8_t v) {
  bf8_t r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (__bf16)(-2.f * (float)v[i]);
  return r;
}

// A list entry is one 64-bit key: the distance's bits above the reference
// index.  Pushed distances are finite and >= +0 (negative values are clamped
// to +0, NaN and inf never pass the filter), so the unsigned key order is the
// (distance, index) order; the empty entry (inf, KB_NONE) is above every
// pushed key and ~0 above it.
__device__ __forceinline__ uint64_t kb_key(float d, int i) {
  return ((uint64_t)__float_as_uint(d) << 32) | (uint32_t)i;
}

// (a, b) := (min, max) and (c, d) := (min, max): two independent exchanges,
// each one 64-bit compare (into vcc, and into an SGPR pair) and four 32-bit
// selects.  The compiler expands the same C++ as a min and a max, a compare
// each.  A 64-bit compare's vcc write takes two wait states before its first
// read (the ones the compiler inserts there): the second compare and one nop.
__device__ __forceinline__ void kb_ce2(uint64_t& a, uint64_t& b, uint64_t& c, uint64_t& d) {
  uint32_t r0, r1, r2, r3, r4, r5, r6, r7;
  uint64_t m;
  asm("v_cmp_lt_u64 vcc, %10, %9\n\t"
      "v_cmp_lt_u64 %8, %12, %11\n\t"
      "s_nop 0\n\t"
      "v_cndmask_b32 %0, %13, %15, vcc\n\t"
      "v_cndmask_b32 %1, %14, %16, vcc\n\t"
      "v_cndmask_b32 %2, %15, %13, vcc\n\t"
      "v_cndmask_b32 %3, %16, %14, vcc\n\t"
      "v_cndmask_b32 %4, %17, %19, %8\n\t"
      "v_cndmask_b32 %5, %18, %20, %8\n\t"
      "v_cndmask_b32 %6, %19, %17, %8\n\t"
      "v_cndmask_b32 %7, %20, %18, %8"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3), "=&v"(r4), "=&v"(r5), "=&v"(r6),
        "=&v"(r7), "=&s"(m)
      : "v"(a), "v"(b), "v"(c), "v"(d),                                  // 9 .. 12
        "v"((uint32_t)a), "v"((uint32_t)(a >> 32)), "v"((uint32_t)b),   // 13 .. 15
        "v"((uint32_t)(b >> 32)), "v"((uint32_t)c), "v"((uint32_t)(c >> 32)),  // 16 .. 18
        "v"((uint32_t)d), "v"((uint32_t)(d >> 32))                        // 19, 20
      : "vcc");
  a = ((uint64_t)r1 << 32) | r0;
  b = ((uint64_t)r3 << 32) | r2;
  c = ((uint64_t)r5 << 32) | r4;
  d = ((uint64_t)r7 << 32) | r6;
}

// a := min(a, b), c := min(c, d), as above
__device__ __forceinline__ void kb_min2(uint64_t& a, uint64_t b, uint64_t& c, uint64_t d) {
  uint32_t r0, r1, r2, r3;
  uint64_t m;
  asm("v_cmp_lt_u64 vcc, %6, %5\n\t"
      "v_cmp_lt_u64 %4, %8, %7\n\t"
      "s_nop 0\n\t"
      "v_cndmask_b32 %0, %9, %11, vcc\n\t"
      "v_cndmask_b32 %1, %10, %12, vcc\n\t"
      "v_cndmask_b32 %2, %13, %15, %4\n\t"
      "v_cndmask_b32 %3, %14, %16, %4"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3), "=&s"(m)
      : "v"(a), "v"(b), "v"(c), "v"(d),
        "v"((uint32_t)a), "v"((uint32_t)(a >> 32)), "v"((uint32_t)b), "v"((uint32_t)(b >> 32)),
        "v"((uint32_t)c), "v"((uint32_t)(c >> 32)), "v"((uint32_t)d), "v"((uint32_t)(d >> 32))
      : "vcc");
  a = ((uint64_t)r1 << 32) | r0;
  c = ((uint64_t)r3 << 32) | r2;
}

// 19-comparator sorting network for 8 keys (checked on every 0/1 input), in
// its six layers of independent exchanges
__device__ __forceinline__ void kb_sort8(uint64_t (&x)[8]) {
  kb_ce2(x[0], x[2], x[1], x[3]); kb_ce2(x[4], x[6], x[5], x[7]);
  kb_ce2(x[0], x[4], x[1], x[5]); kb_ce2(x[2], x[6], x[3], x[7]);
  kb_ce2(x[0], x[1], x[2], x[3]); kb_ce2(x[4], x[5], x[6], x[7]);
  kb_ce2(x[2], x[4], x[3], x[5]);
  kb_ce2(x[1], x[4], x[3], x[6]);
  kb_ce2(x[1], x[2], x[3], x[4]);
  uint64_t t = 0;
  kb_ce2(x[5], x[6], t, t);  // the layer's third exchange, paired with a no-op
}

// l := the KC smallest of the sorted list l and the NB <= KC sorted keys x,
// sorted.  The list's last NB take the minimum with x reversed (an ascending
// and a descending run: the KC smallest, as a bitonic sequence), then
// log2(KC) half-cleaner stages sort it.
template <int KC, int NB>
__device__ __forceinline__ void kb_merge(uint64_t (&l)[KC], const uint64_t (&x)[NB]) {
  static_assert(NB % 2 == 0 && NB <= KC, "pairs of exchanges");
#pragma unroll
  for (int i = 0; i < NB; i += 2) kb_min2(l[KC - NB + i], x[NB - 1 - i], l[KC - NB + 1 + i], x[NB - 2 - i]);
#pragma unroll
  for (int st = KC / 2; st > 0; st >>= 1) {
    // the stage's KC/2 exchanges (i, i + st), i without bit st, two at a time
#pragma unroll
    for (int p = 0; p < KC / 2; p += 2) {
      const int i0 = (p / st) * 2 * st + p % st, i1 = ((p + 1) / st) * 2 * st + (p + 1) % st;
      kb_ce2(l[i0], l[i0 + st], l[i1], l[i1 + st]);
    }
  }
}

// The next float above x (x finite; +inf and NaN give +inf): d < kb_next_up(x)
// holds exactly when d <= x.
__device__ __forceinline__ float kb_next_up(float x) {
  if (!(x < Lim<float>::inf())) return Lim<float>::inf();
  if (x == 0.f) return __uint_as_float(1u);
  const uint32_t b = __float_as_uint(x);
  return __uint_as_float(x > 0.f ? b + 1u : b - 1u);
}

// s := the KB_TK smallest of the sorted s and one more value (sorted)
__device__ __forceinline__ void kb_tk_insert(float (&s)[KB_TK], float d) {
#pragma unroll
  for (int i = KB_TK - 1; i > 0; --i) s[i] = d < s[i - 1] ? s[i - 1] : (d < s[i] ? d : s[i]);
  s[0] = d < s[0] ? d : s[0];
}

// The sampled bound of query position q of cloud n, as the filter limit: the
// KB_TK-th smallest of its KB_TP sorted part lists (a bitonic merge of each
// into the running KB_TK), moved one float up, so d < limit exactly when
// d <= the bound.
__device__ __forceinline__ float kb_tau(const float* __restrict__ taup, int n, int P1, int q) {
  const float* __restrict__ tq = taup + (size_t)n * KB_TP * KB_TK * P1 + q;
  float t[KB_TK];
#pragma unroll
  for (int i = 0; i < KB_TK; ++i) t[i] = tq[(size_t)i * P1];
#pragma unroll 1
  for (int pp = 1; pp < KB_TP; ++pp) {
    float u[KB_TK];
#pragma unroll
    for (int i = 0; i < KB_TK; ++i) u[i] = tq[((size_t)pp * KB_TK + i) * P1];
#pragma unroll
    for (int i = 0; i < KB_TK; ++i) t[i] = fminf(t[i], u[KB_TK - 1 - i]);
#pragma unroll
    for (int st = KB_TK / 2; st > 0; st >>= 1)
#pragma unroll
      for (int i = 0; i < KB_TK; ++i)
        if (!(i & st)) {
          const float lo = fminf(t[i], t[i + st]), hi = fmaxf(t[i], t[i + st]);
          t[i] = lo;
          t[i + st] = hi;
        }
  }
  return kb_next_up(t[KB_TK - 1]);
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
// (two waves a SIMD: one wave's MFMA chain runs under the other's selection
// work; the register budget of 256 is held with a few spills outside the tile
// loop's hot path)
template <int KS, bool HALF, int KC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void knn_bf16_slice_kernel(
    const __bf16* __restrict__ p1, const __bf16* __restrict__ p2, const int64_t* __restrict__ len1,
    const int64_t* __restrict__ len2, int P1, int P2, int D, int K, int nqb, int slices,
    const float* __restrict__ qn, const float* __restrict__ rn, uint64_t* __restrict__ part,
    const int32_t* __restrict__ qlist, const int32_t* __restrict__ qcount) {
  __shared__ uint64_t s_q[KB_WAVES][KB_QCAP][64];
  // a tile's reference rows (D bfloat16 each, rows 2D + 16 bytes apart so a
  // half-wave's 16-byte reads of 16 rows fall in distinct banks) and their
  // norms, double-buffered: the workgroup loads each tile once for its waves
  constexpr int RS = 2 * KB_DMAX + 16;
  __shared__ __align__(16) char s_rows[2][KB_T * RS];
  __shared__ float s_rn[2][KB_T];

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
  // Positions: queries themselves, or (qlist: the rerun of the rows the
  // candidate pass under the sampled bound could not settle) entries of
  // cloud n's list of qcount[n] rows.
  const int npos = qlist ? qcount[n] : (int)l1;
  if (qlist && qb * KB_QW >= npos) return;  // the whole workgroup past the list
  const int32_t* __restrict__ ql = qlist ? qlist + (size_t)n * P1 : nullptr;
  auto query_at = [&](int pos) { return ql ? ql[min(pos, npos - 1)] : min(pos, P1 - 1); };
  const int qw = qb * KB_QW + 64 * w;  // the wave's blocks: positions qw + 32 b + column
  const int q = qw + lane;             // this lane's position after the swap: block h, column j

  // k-steps of the MFMA chain: KS of dims, and the norms' step -- the upper
  // half of the last dims step when D % 16 == 8 (lanes h = 1 there lie past
  // D), else a step of its own (in its lower half)
  constexpr int KX = HALF ? KS : KS + 1, XS = KX - 1, XH = HALF ? 1 : 0;
  // column operands of both blocks: query qw + 32 b + j, dims 16s + 8h .. + 7
  // times -2 (zero past D), then the query's norm pieces
  bf8_t bq0[KX], bq1[KX];
  {
    const int c0 = query_at(qw + j), c1 = query_at(qw + 32 + j);
    const __bf16* __restrict__ qp0 = p1 + ((size_t)n * P1 + c0) * D;
    const __bf16* __restrict__ qp1 = p1 + ((size_t)n * P1 + c1) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int d0 = 16 * s + 8 * h;
      bq0[s] = d0 < D ? kb_neg2(*reinterpret_cast<const bf8_t*>(qp0 + d0)) : bf8_t{};
      bq1[s] = d0 < D ? kb_neg2(*reinterpret_cast<const bf8_t*>(qp1 + d0)) : bf8_t{};
    }
    const bf8_t x0 = kb_norm_operand(qn[(size_t)n * kb_pad(P1) + c0], false);
    const bf8_t x1 = kb_norm_operand(qn[(size_t)n * kb_pad(P1) + c1], false);
    bq0[XS] = h == XH ? x0 : (HALF ? bq0[XS] : bf8_t{});
    bq1[XS] = h == XH ? x1 : (HALF ? bq1[XS] : bf8_t{});
  }
  const __bf16* __restrict__ rb = p2 + (size_t)n * P2 * D;
  const float* __restrict__ rr = rn + (size_t)n * kb_pad(P2);

  // the slice's tiles
  const int ntiles = (L2 + KB_T - 1) / KB_T;
  const int tps = (ntiles + slices - 1) / slices;
  const int t0 = min(sl * tps, ntiles), t1 = min(ntiles, t0 + tps);


  uint64_t lk[KC];  // this lane's list, ascending keys
#pragma unroll
  for (int s = 0; s < KC; ++s) lk[s] = kb_key(Lim<float>::inf(), KB_NONE);
  int nq_ = 0;  // queued candidates of this lane
  // merge the queue into the list 8 entries at a time (slots past the lane's
  // count read as ~0): a sorting network, then a bitonic merge, all in
  // registers with fixed indices; a stale entry (pushed against an older
  // threshold) simply falls off the end
  auto drain = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int g8 = 0; g8 < KB_QCAP / 8; ++g8) {
      if (__ballot(nq_ > 8 * g8) == 0) break;
      uint64_t x[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint64_t e = s_q[w][8 * g8 + i][lane];
        x[i] = 8 * g8 + i < nq_ ? e : ~0ull;
      }
      kb_sort8(x);
      kb_merge<KC, 8>(lk, x);
    }
    nq_ = 0;
  };

  // Staging of tile t: thread tid loads row tid / 8 (clamped into [0, L2);
  // a tile past the slice re-reads the last), 16-byte chunks tid % 8 and
  // tid % 8 + 8 of its D / 8, and threads < 32 the norm of row tid (+inf past
  // L2: the row's distances are NaN and never pass the filter).  The loads go
  // to registers one tile ahead and to LDS after the tile's work.
  const int rrow = tid >> 3, rch = tid & 7, rstride = 2 * D + 16;
  bf8_t st0, st1;
  float stn;
  auto stage_load = [&](int t) __attribute__((always_inline)) {
    const int base = min(t, ntiles - 1) * KB_T;
    const __bf16* __restrict__ ra = rb + (size_t)min(base + rrow, L2 - 1) * D;
    st0 = 8 * rch < D ? *reinterpret_cast<const bf8_t*>(ra + 8 * rch) : bf8_t{};
    st1 = 8 * rch + 64 < D ? *reinterpret_cast<const bf8_t*>(ra + 8 * rch + 64) : bf8_t{};
    stn = tid < KB_T ? (base + tid < L2 ? rr[min(base + tid, L2 - 1)] : Lim<float>::inf()) : 0.f;
  };
  auto stage_store = [&](int b) __attribute__((always_inline)) {
    char* __restrict__ dst = s_rows[b] + rrow * rstride;
    if (8 * rch < D) *reinterpret_cast<bf8_t*>(dst + 16 * rch) = st0;
    if (8 * rch + 64 < D) *reinterpret_cast<bf8_t*>(dst + 16 * rch + 128) = st1;
    if (tid < KB_T) s_rn[b][tid] = stn;
  };
  // Tile t (staged in buffer b): multiply, swap, filter, queue.  Row operand
  // for this lane: row j, dims 16s + 8h .. + 7 (a half past D re-reads the
  // step's lower half and is replaced by the norm operand).
  auto tile = [&](int t, int b) __attribute__((always_inline)) {
    const int base = t * KB_T;
    const char* __restrict__ src = s_rows[b] + j * rstride;
    bf8_t a[KX];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int d0 = (HALF && s == KS - 1) ? 16 * s : 16 * s + 8 * h;
      a[s] = *reinterpret_cast<const bf8_t*>(src + 2 * d0);
    }
    {
      const bf8_t xr = kb_norm_operand(s_rn[b][j], true);
      a[XS] = h == XH ? xr : (HALF ? a[XS] : bf8_t{});
    }
    f16v_t acc0 = {}, acc1 = {};
#pragma unroll
    for (int s = 0; s < KX; ++s) {
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
    // Two halves of 16 rows (8-row groups 2c, 2c + 1).  The filter compares
    // the unclamped value (a negative one passes it, and the pushed value is
    // clamped at 0).
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const float thr = __uint_as_float((uint32_t)(lk[KC - 1] >> 32));
      float dv[16];
      uint32_t m = 0;  // bit 15 - v: row 16c + v is below the list's end
#pragma unroll
      for (int gg = 0; gg < 2; ++gg) {
        const int g = 2 * c + gg;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          float d4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float d = hh ? acc1[4 * g + e] : acc0[4 * g + e];
            dv[8 * gg + 4 * hh + e] = d;  // row 16c + 8gg + 4hh + e
            d4[e] = d;
          }
          m = push_lt4(m, d4[0], d4[1], d4[2], d4[3], thr);
        }
      }
      if (__ballot(m != 0) != 0) {  // some lane has a candidate in these rows
        if (__ballot(nq_ + __builtin_popcount(m) > KB_QCAP) != 0) drain();  // queues within capacity
        // only the set bits: the wave pays max-over-lanes(candidates), not 16
        // rows of branches (thr may predate a drain: a stale entry is merged
        // and falls off the list's end; the queue's order is immaterial)
        while (m) {
          const int v = 15 - __builtin_ctz(m);
          m &= m - 1;
          s_q[w][nq_][lane] = kb_key(fmaxf(kb_sel16(dv, v), 0.f), base + 16 * c + v);
          ++nq_;
        }
      }
    }
  };
  if (t0 < t1) {
    stage_load(t0);
    stage_store(0);
  }
  for (int t = t0; t < t1; ++t) {
    const int b = (t - t0) & 1;
    __syncthreads();  // tile t staged; every wave is past its reads of buffer b ^ 1
    if (t + 1 < t1) stage_load(t + 1);
    tile(t, b);
    if (t + 1 < t1) stage_store(b ^ 1);
  }
  drain();

  // the first K entries of this lane's list
  if (q < npos) {
    // entry s of (cloud n, slice sl) for all queries is one run of P1 keys:
    // a wave's stores are 64 consecutive keys
    uint64_t* __restrict__ out = part + (size_t)(n * slices + sl) * K * P1 + q;
#pragma unroll
    for (int s = 0; s < KC; ++s)
      if (s < K) out[(size_t)s * P1] = lk[s];
  }
}

// The sampled bound's parts: workgroup (cloud n, part pt, query block qb)
// runs the slice kernel's products over tiles (pt + KB_TP k) * stride,
// k < KB_TK = KB_TS / KB_TP, stride = ntiles / KB_TS, and keeps each query's
// smallest distance of every tile: the part's KB_TK tile minima, sorted
// (+inf when none), stored [n][pt][i][query].  The KB_TK-th smallest of a
// query's KB_TS tile minima is a sampled distance with at least KB_TK sampled
// distances at or below it.  The workgroup stages its KB_TK tiles in LDS at
// once (every load in flight together), then each wave runs them back to
// back.  Workgroup 0 also clears the rerun counts.
template <int KS, bool HALF>
__global__ __launch_bounds__(256) void knn_bf16_tau_kernel(
    const __bf16* __restrict__ p1, const __bf16* __restrict__ p2, const int64_t* __restrict__ len1,
    const int64_t* __restrict__ len2, int N, int P1, int P2, int K, int nqb,
    const float* __restrict__ qn, const float* __restrict__ rn, float* __restrict__ taup,
    int32_t* __restrict__ rcount) {
  static_assert(KB_TS / KB_TP == KB_TK, "a part is KB_TK tiles");
  constexpr int D = 16 * KS - (HALF ? 8 : 0);  // the dimension (the dispatch's choice of KS, HALF)
  constexpr int RS = 2 * D + 16, NR = KB_TK * KB_T;  // row stride, rows staged
  __shared__ __align__(16) char s_rows[NR * RS];
  __shared__ bf8_t s_rx[NR];
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < N; i += 256) rcount[i] = 0;
  const int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int qb = lb % nqb, ns = lb / nqb;
  const int pt = ns % KB_TP, n = ns / KB_TP;
  int64_t l1 = len1[n], l2 = len2[n];
  l1 = l1 < 0 ? 0 : (l1 > P1 ? P1 : l1);
  l2 = l2 < 0 ? 0 : (l2 > P2 ? P2 : l2);
  const int L2 = (int)l2;
  const int tid = threadIdx.x, w = wave_id(), lane = lane_id(), j = lane & 31, h = lane >> 5;
  const int qw = qb * KB_QW + 64 * w;
  const int q = qw + lane;
  constexpr int KX = HALF ? KS : KS + 1, XS = KX - 1, XH = HALF ? 1 : 0;
  float s[KB_TK];
#pragma unroll
  for (int i = 0; i < KB_TK; ++i) s[i] = Lim<float>::inf();
  const int ntiles = (L2 + KB_T - 1) / KB_T;
  if (kb_sampled(L2, K)) {  // workgroup-uniform
    const __bf16* __restrict__ rb = p2 + (size_t)n * P2 * D;
    const float* __restrict__ rr = rn + (size_t)n * kb_pad(P2);
    const int stride = ntiles / KB_TS;
    // staging: tile k's row r (thread tid: r = tid / 8, 16-byte chunks
    // tid % 8 and tid % 8 + 8 of every tile; thread tid: the norm of staged
    // row tid); the sampled tiles lie inside the cloud
    const int rrow = tid >> 3, rch = tid & 7;
    {
      bf8_t st[KB_TK][2];
#pragma unroll
      for (int k = 0; k < KB_TK; ++k) {
        const __bf16* __restrict__ ra = rb + ((size_t)(pt + KB_TP * k) * stride * KB_T + rrow) * D;
        st[k][0] = 8 * rch < D ? *reinterpret_cast<const bf8_t*>(ra + 8 * rch) : bf8_t{};
        st[k][1] = 8 * rch + 64 < D ? *reinterpret_cast<const bf8_t*>(ra + 8 * rch + 64) : bf8_t{};
      }
      const float nrm = rr[(size_t)(pt + KB_TP * (tid / KB_T)) * stride * KB_T + tid % KB_T];
#pragma unroll
      for (int k = 0; k < KB_TK; ++k) {
        char* __restrict__ dst = s_rows + (k * KB_T + rrow) * RS;
        if (8 * rch < D) *reinterpret_cast<bf8_t*>(dst + 16 * rch) = st[k][0];
        if (8 * rch + 64 < D) *reinterpret_cast<bf8_t*>(dst + 16 * rch + 128) = st[k][1];
      }
      s_rx[tid] = kb_norm_operand(nrm, true);
    }
    bf8_t bq0[KX], bq1[KX];
    {
      const int c0 = min(qw + j, P1 - 1), c1 = min(qw + 32 + j, P1 - 1);
      const __bf16* __restrict__ qp0 = p1 + ((size_t)n * P1 + c0) * D;
      const __bf16* __restrict__ qp1 = p1 + ((size_t)n * P1 + c1) * D;
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        const int d0 = 16 * st + 8 * h;
        bq0[st] = d0 < D ? kb_neg2(*reinterpret_cast<const bf8_t*>(qp0 + d0)) : bf8_t{};
        bq1[st] = d0 < D ? kb_neg2(*reinterpret_cast<const bf8_t*>(qp1 + d0)) : bf8_t{};
      }
      const bf8_t x0 = kb_norm_operand(qn[(size_t)n * kb_pad(P1) + c0], false);
      const bf8_t x1 = kb_norm_operand(qn[(size_t)n * kb_pad(P1) + c1], false);
      bq0[XS] = h == XH ? x0 : (HALF ? bq0[XS] : bf8_t{});
      bq1[XS] = h == XH ? x1 : (HALF ? bq1[XS] : bf8_t{});
    }
    __syncthreads();
#pragma unroll 1
    for (int k = 0; k < KB_TK; ++k) {
      const char* __restrict__ src = s_rows + (k * KB_T + j) * RS;
      bf8_t a[KX];
#pragma unroll
      for (int st = 0; st < KS - (HALF ? 1 : 0); ++st)
        a[st] = *reinterpret_cast<const bf8_t*>(src + 2 * (16 * st + 8 * h));
      // the norm step as in the candidate pass
      a[XS] = *(HALF && h == 0 ? reinterpret_cast<const bf8_t*>(src + 2 * 16 * (KS - 1))
                               : &s_rx[k * KB_T + j]);
      f16v_t acc0 = {}, acc1 = {};
#pragma unroll
      for (int st = 0; st < KX; ++st) {
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[st], bq0[st], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[st], bq1[st], acc1, 0, 0, 0);
      }
      // the tile's smallest distance for the lane's query: lane l holds 16
      // rows of column l % 32 of each block, its partner l ^ 32 the other 16,
      // combined by one swap
      float m0 = acc0[0], m1 = acc1[0];
#pragma unroll
      for (int v = 1; v < 16; ++v) {
        m0 = fminf(m0, acc0[v]);
        m1 = fminf(m1, acc1[v]);
      }
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(m0), __float_as_uint(m1), false, false);
      kb_tk_insert(s, fminf(__uint_as_float(r[0]), __uint_as_float(r[1])));
    }
  }
  if (q < P1 && q < l1) {
    float* __restrict__ out = taup + ((size_t)(n * KB_TP + pt) * KB_TK) * P1 + q;
#pragma unroll
    for (int i = 0; i < KB_TK; ++i) out[(size_t)i * P1] = s[i];
  }
}

// Work split of the candidate pass: query blocks of 256 and up to
// KB_CMAX_SLICES reference slices, about three workgroups a CU (as many as
// are resident at once).
static KbPlan kb_cplan(int64_t N, int64_t P1, int64_t P2) {
  KbPlan p;
  p.nqb = (int)((P1 + KB_QW - 1) / KB_QW);
  const int64_t wgs = N * (int64_t)p.nqb;
  int64_t s = wgs > 0 ? (768 + wgs - 1) / wgs : 1;
  const int64_t tiles = (P2 + KB_T - 1) / KB_T;
  s = std::min<int64_t>(s, std::max<int64_t>(1, tiles / 16));  // at least 16 tiles a slice
  p.slices = (int)std::max<int64_t>(1, std::min<int64_t>(s, KB_CMAX_SLICES));
  return p;
}

// The candidate pass under the sampled bound.  Workgroup (cloud n, slice sl,
// query block qb) stages the slice's tiles in LDS and runs the slice
// kernel's MFMA chain, but keeps no list: every distance at or below its
// query's bound is stored at once, as a 64-bit key, in the region of (query,
// slice) -- KB_CAP slots, which the half-wave h = 0 fills upwards from the
// first and h = 1 downwards from the last.  No swap is needed: lane (h, j)
// tests its block-0 column (position qw + j) against that query's bound and
// its block-1 column (qw + 32 + j) against that one's.  Counts run on past the
// capacity (the last slot is overwritten); the merge sends such a query, and
// one left with fewer than min(K, lengths2) candidates, to the exact pass.
template <int KS, bool HALF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void knn_bf16_cand_kernel(
    const __bf16* __restrict__ p1, const __bf16* __restrict__ p2, const int64_t* __restrict__ len1,
    const int64_t* __restrict__ len2, int P1, int P2, int K, int nqb, int slices,
    const float* __restrict__ qn, const float* __restrict__ rn, const float* __restrict__ taup,
    uint64_t* __restrict__ cand, int32_t* __restrict__ ccount) {
  constexpr int D = 16 * KS - (HALF ? 8 : 0);  // the dimension (the dispatch's choice of KS, HALF)
  constexpr int RS = 2 * KB_DMAX + 16;
  // two tiles a stage (one barrier for both), double-buffered
  constexpr int TC = 2, CR = TC * KB_T;
  __shared__ __align__(16) char s_rows[2][CR * RS];
  __shared__ bf8_t s_rx[2][CR];  // the rows' norm operands
  const int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int qb = lb % nqb, ns = lb / nqb;
  const int sl = ns % slices, n = ns / slices;
  int64_t l1 = len1[n], l2 = len2[n];
  l1 = l1 < 0 ? 0 : (l1 > P1 ? P1 : l1);
  l2 = l2 < 0 ? 0 : (l2 > P2 ? P2 : l2);
  // the whole workgroup past the cloud's queries, or a cloud without the
  // bound (its rows all take the exact pass; the merge lists them)
  if (qb * KB_QW >= l1 || !kb_sampled(l2, K)) return;
  const int L2 = (int)l2;
  const int tid = threadIdx.x, w = wave_id(), lane = lane_id(), j = lane & 31, h = lane >> 5;
  const int qw = qb * KB_QW + 64 * w;

  constexpr int KX = HALF ? KS : KS + 1, XS = KX - 1, XH = HALF ? 1 : 0;
  bf8_t bq0[KX], bq1[KX];
  {
    const int c0 = min(qw + j, P1 - 1), c1 = min(qw + 32 + j, P1 - 1);
    const __bf16* __restrict__ qp0 = p1 + ((size_t)n * P1 + c0) * D;
    const __bf16* __restrict__ qp1 = p1 + ((size_t)n * P1 + c1) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int d0 = 16 * s + 8 * h;
      bq0[s] = d0 < D ? kb_neg2(*reinterpret_cast<const bf8_t*>(qp0 + d0)) : bf8_t{};
      bq1[s] = d0 < D ? kb_neg2(*reinterpret_cast<const bf8_t*>(qp1 + d0)) : bf8_t{};
    }
    const bf8_t x0 = kb_norm_operand(qn[(size_t)n * kb_pad(P1) + c0], false);
    const bf8_t x1 = kb_norm_operand(qn[(size_t)n * kb_pad(P1) + c1], false);
    bq0[XS] = h == XH ? x0 : (HALF ? bq0[XS] : bf8_t{});
    bq1[XS] = h == XH ? x1 : (HALF ? bq1[XS] : bf8_t{});
  }
  const __bf16* __restrict__ rb = p2 + (size_t)n * P2 * D;
  const float* __restrict__ rr = rn + (size_t)n * kb_pad(P2);
  const int ntiles = (L2 + KB_T - 1) / KB_T;
  const int tps = (ntiles + slices - 1) / slices;
  const int t0 = min(sl * tps, ntiles), t1 = min(ntiles, t0 + tps);

  // Bounds: lane l computes that of position qw + l (-inf past the cloud's
  // queries: nothing passes it); the swap hands lane (h, j) those of qw + j
  // and qw + 32 + j.
  const float lim = qw + lane < l1 ? kb_tau(taup, n, P1, qw + lane) : -Lim<float>::inf();
  const auto lr = __builtin_amdgcn_permlane32_swap(__float_as_uint(lim), __float_as_uint(lim), false, false);
  const float lim0 = __uint_as_float(lr[0]), lim1 = __uint_as_float(lr[1]);
  // The wave's regions: (position qw + x, slice sl) starts x * rstep bytes
  // past wbase; this lane's slot c of its half lies o + e8 * c bytes past it.
  char* __restrict__ wbase =
      reinterpret_cast<char*>(cand + (((size_t)n * P1 + qw) * slices + sl) * KB_CAP);
  const int rstep = slices * KB_CAP * 8, e8 = h ? -8 : 8;
  const int o0 = j * rstep + (h ? (KB_CAP - 1) * 8 : 0), o1 = o0 + 32 * rstep;
  int c0 = 0, c1 = 0;  // candidates of this lane's half for its two queries
  // A tile's 32 distances per lane are tested into one 32-bit mask (bit
  // 31 - v: acc0[v] for v < 16, else acc1[v - 16], is at or below its
  // query's bound), without branches; then each lane stores its candidates
  // one at a time (the wave loops max-over-lanes times, ~1.4 a tile), the
  // value picked by a select tree.  A negative distance, stored as +0, is
  // clamped on its bits; NaN (rows past the cloud) never passes.
  auto filter = [&](const f16v_t& acc0, const f16v_t& acc1, int rb) __attribute__((always_inline)) {
    // The compares are inline asm, after which the compiler would not wait
    // for the MFMA results: a compiler-visible read of both accumulators
    // (the last written) comes first, and the mask depends on it (its bit
    // is shifted out).
    uint32_t m = __builtin_isnan(acc0[15] + acc1[15]) ? 1u : 0u;
#pragma unroll
    for (int g = 0; g < 4; ++g)
      m = push_lt4(m, acc0[4 * g], acc0[4 * g + 1], acc0[4 * g + 2], acc0[4 * g + 3], lim0);
#pragma unroll
    for (int g = 0; g < 4; ++g)
      m = push_lt4(m, acc1[4 * g], acc1[4 * g + 1], acc1[4 * g + 2], acc1[4 * g + 3], lim1);
    if (__ballot(m != 0) == 0) return;
    while (m) {
      const int v = 31 - __builtin_ctz(m);
      m &= m - 1;
      const uint32_t m4 = bit_mask(v, 4);
      float e[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) e[i] = csel(m4, acc0[i], acc1[i]);
      const float d = kb_sel16(e, v & 15);
      const bool second = v >= 16;
      const int c = second ? c1 : c0, o = second ? o1 : o0;
      const uint32_t db = (uint32_t)max((int32_t)__float_as_uint(d), 0);
      *reinterpret_cast<uint64_t*>(wbase + (uint32_t)(o + e8 * min(c, KB_CAP - 1))) =
          ((uint64_t)db << 32) | (uint32_t)(rb + 8 * ((v >> 2) & 3) + (v & 3));
      c0 += second ? 0 : 1;
      c1 += second ? 1 : 0;
    }
  };

  // Staging of tiles t, t + 1 as in the slice kernel (thread tid: rows
  // tid / 8 and tid / 8 + 32); threads < 64 also turn their row's norm into
  // its MFMA operand.
  const int rrow = tid >> 3, rch = tid & 7;
  constexpr int rstride = 2 * D + 16;
  bf8_t st0, st1, st2, st3;
  float stn;
  auto stage_load = [&](int t) __attribute__((always_inline)) {
    const int base = min(t, ntiles - 1) * KB_T;
    const __bf16* __restrict__ ra = rb + (size_t)min(base + rrow, L2 - 1) * D;
    const __bf16* __restrict__ rc = rb + (size_t)min(base + 32 + rrow, L2 - 1) * D;
    st0 = 8 * rch < D ? *reinterpret_cast<const bf8_t*>(ra + 8 * rch) : bf8_t{};
    st1 = 8 * rch + 64 < D ? *reinterpret_cast<const bf8_t*>(ra + 8 * rch + 64) : bf8_t{};
    st2 = 8 * rch < D ? *reinterpret_cast<const bf8_t*>(rc + 8 * rch) : bf8_t{};
    st3 = 8 * rch + 64 < D ? *reinterpret_cast<const bf8_t*>(rc + 8 * rch + 64) : bf8_t{};
    stn = tid < CR ? (base + tid < L2 ? rr[min(base + tid, L2 - 1)] : Lim<float>::inf()) : 0.f;
  };
  auto stage_store = [&](int b) __attribute__((always_inline)) {
    char* __restrict__ dst = s_rows[b] + rrow * rstride;
    if (8 * rch < D) *reinterpret_cast<bf8_t*>(dst + 16 * rch) = st0;
    if (8 * rch + 64 < D) *reinterpret_cast<bf8_t*>(dst + 16 * rch + 128) = st1;
    if (8 * rch < D) *reinterpret_cast<bf8_t*>(dst + 32 * rstride + 16 * rch) = st2;
    if (8 * rch + 64 < D) *reinterpret_cast<bf8_t*>(dst + 32 * rstride + 16 * rch + 128) = st3;
    if (tid < CR) s_rx[b][tid] = kb_norm_operand(stn, true);
  };
  // tile tt of the stage in buffer b times both query blocks; the operand
  // reads run three k-steps ahead of the MFMAs (the schedule is pinned: left
  // alone, the compiler waits for each read right before its MFMAs)
  auto mma = [&](int b, int tt, f16v_t& acc0, f16v_t& acc1) __attribute__((always_inline)) {
    const char* __restrict__ src = s_rows[b] + (32 * tt + j) * rstride;
    bf8_t a[KX];
#pragma unroll
    for (int s = 0; s < KS - (HALF ? 1 : 0); ++s)
      a[s] = *reinterpret_cast<const bf8_t*>(src + 2 * (16 * s + 8 * h));
    // the norm step: without HALF both halves read the operand (the query
    // operand's upper half is zero there); with HALF the lower half is the
    // last dims step's lower half
    a[XS] = *(HALF && h == 0 ? reinterpret_cast<const bf8_t*>(src + 2 * 16 * (KS - 1))
                             : &s_rx[b][32 * tt + j]);
    acc0 = f16v_t{};
    acc1 = f16v_t{};
#pragma unroll
    for (int s = 0; s < KX; ++s) {
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s], bq0[s], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s], bq1[s], acc1, 0, 0, 0);
    }
    constexpr int AH = KX < 3 ? KX : 3;  // reads ahead
    __builtin_amdgcn_sched_group_barrier(0x100, AH, 0);  // DS reads
#pragma unroll
    for (int s = 0; s < KX - AH; ++s) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * AH, 0);
  };
  if (t0 < t1) {
    stage_load(t0);
    stage_store(0);
  }
  for (int tc = t0; tc < t1; tc += TC) {
    const int b = ((tc - t0) / TC) & 1;
    __syncthreads();  // stage tc staged; every wave is past its reads of buffer b ^ 1
    if (tc + TC < t1) stage_load(tc + TC);
#pragma unroll
    for (int tt = 0; tt < TC; ++tt) {
      const int t = tc + tt;
      if (t < t1) {
        f16v_t acc0, acc1;
        mma(b, tt, acc0, acc1);
        // The next stage goes to LDS before this tile's candidates are
        // stored: the wait for its loads then covers no store of this tile.
        if (tt == 0 && tc + TC < t1) stage_store(b ^ 1);
        // acc0[v], acc1[v]: row 8 (v / 4) + 4 h + v % 4 of the tile
        filter(acc0, acc1, __builtin_amdgcn_readfirstlane(t * KB_T) + 4 * h);
      }
    }
  }
  // counts of (position, slice, half)
  const size_t cr = ((size_t)n * P1 + qw) * slices + sl;
  if (qw + j < l1) ccount[(cr + (size_t)j * slices) * 2 + h] = c0;
  if (qw + 32 + j < l1) ccount[(cr + (size_t)(32 + j) * slices) * 2 + h] = c1;
}

// LDS written by some lanes of a wave, then read by others
__device__ __forceinline__ void kb_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Wave reductions and scans over DPP (every lane active).
template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint32_t kb_dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWMASK, 0xf, true);
}
// the minimum (MAX: maximum) over the wave, uniform
template <bool MAX>
__device__ __forceinline__ uint32_t kb_wave_uext(uint32_t v) {
  auto f = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
  // quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror: every lane
  // holds its row's result; row_bcast:15 into rows 1, 3 and row_bcast:31 into
  // rows 2, 3 (masked-off rows read 0, which a maximum ignores; a minimum
  // skips those steps' effect through v itself)
  v = f(v, __builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xf, 0xf, false));
  v = f(v, __builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xf, 0xf, false));
  v = f(v, __builtin_amdgcn_update_dpp((int)v, (int)v, 0x141, 0xf, 0xf, false));
  v = f(v, __builtin_amdgcn_update_dpp((int)v, (int)v, 0x140, 0xf, 0xf, false));
  v = f(v, __builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xa, 0xf, false));
  v = f(v, __builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xc, 0xf, false));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
// inclusive prefix sum over lanes: row_shr 1, 2, 4, 8 within each row of 16
// (lanes past the row's start read 0), then the rows' totals by row_bcast:15
// into rows 1, 3 and row_bcast:31 into rows 2, 3
__device__ __forceinline__ uint32_t kb_wave_scan(uint32_t v) {
  v += kb_dpp<0x111, 0xf>(v);
  v += kb_dpp<0x112, 0xf>(v);
  v += kb_dpp<0x114, 0xf>(v);
  v += kb_dpp<0x118, 0xf>(v);
  v += kb_dpp<0x142, 0xa>(v);
  v += kb_dpp<0x143, 0xc>(v);
  return v;
}

// The exact K smallest of a row's candidate keys, held NK to a lane (~0
// where none), total of them, for the candidate pass's merge: above 64
// candidates a 64-bin histogram of the distances, linear between their
// minimum and maximum (a monotone map), finds the bin B of the K-th smallest
// -- only candidates in bins <= B can be among the K, and at least K are.
// Those are gathered in sel (up to KB_SEL, past which each lane has a spare
// slot; false when more: the row is rerun exactly); as keys are distinct
// (the index is part of the key), each one's rank among them is its output
// slot.  Slots past the candidates (fewer than K references) are (0, 0).
constexpr int KB_SEL = 512;
template <int NK>
__device__ __forceinline__ bool kb_select(const uint64_t (&key)[NK], int total, int K,
                                          uint32_t* __restrict__ hist,
                                          uint64_t* __restrict__ sel, int64_t* __restrict__ io,
                                          __bf16* __restrict__ dout) {
  constexpr int NB = 64;
  const int lane = lane_id();
  const uint64_t none = ~0ull;
  // the distance bits (a candidate's distance is >= +0, so its bits order as
  // the distance does; the empty key's are ~0)
  uint32_t db[NK];
#pragma unroll
  for (int s = 0; s < NK; ++s) db[s] = (uint32_t)(key[s] >> 32);
  bool all = true;  // every candidate is gathered
  uint32_t bsel = NB, lo = 0;
  float mn = 0.f, scale = 0.f;
  if (total > 64) {
    uint32_t a = ~0u, b = 0;
#pragma unroll
    for (int s = 0; s < NK; ++s) {
      a = min(a, db[s]);
      b = max(b, db[s] != ~0u ? db[s] : 0u);
    }
    lo = kb_wave_uext<false>(a);
    const uint32_t hi = kb_wave_uext<true>(b);
    mn = __uint_as_float(lo);
    scale = (float)NB / (__uint_as_float(hi) - mn);
    if (scale < Lim<float>::inf()) {  // else one value (or a tiny span): gather all
      all = false;
      hist[lane] = 0;
      kb_wave_sync();
#pragma unroll
      for (int s = 0; s < NK; ++s)
        if (db[s] != ~0u) atomicAdd(&hist[min(NB - 1, (int)((__uint_as_float(db[s]) - mn) * scale))], 1u);
      kb_wave_sync();
      const uint32_t c = kb_wave_scan(hist[lane]);  // candidates in bins <= lane
      const uint64_t reach = __ballot(c >= (uint32_t)K);
      bsel = reach ? (uint32_t)__builtin_ctzll(reach) : NB;
    }
  }
  // the candidates that can be among the K: this lane's count, its offset
  // among the wave's, then its keys in order
  bool take[NK];
  uint32_t q = 0;
#pragma unroll
  for (int s = 0; s < NK; ++s) {
    take[s] = db[s] != ~0u &&
              (all || (uint32_t)min(NB - 1, (int)((__uint_as_float(db[s]) - mn) * scale)) <= bsel);
    q += take[s] ? 1u : 0u;
  }
  const uint32_t incl = kb_wave_scan(q);
  const int nsel = (int)__builtin_amdgcn_readlane((int)incl, 63);
  if (nsel > KB_SEL) return false;  // a mass of equal or nearly equal distances
  uint32_t at = incl - q;
#pragma unroll
  for (int s = 0; s < NK; ++s) {
    sel[take[s] ? at : KB_SEL + lane] = key[s];
    at += take[s] ? 1u : 0u;
  }
  kb_wave_sync();
  for (int c = 0; c < nsel; c += 64) {
    const int i = c + lane;
    const uint64_t y = i < nsel ? sel[i] : none;
    int rank = 0;
#pragma unroll 4
    for (int x = 0; x < nsel; ++x) rank += sel[x] < y ? 1 : 0;
    if (i < nsel && rank < K) {
      io[rank] = (int64_t)(uint32_t)y;
      dout[rank] = (__bf16)__uint_as_float((uint32_t)(y >> 32));
    }
  }
  if (lane >= nsel && lane < K) {
    io[lane] = 0;
    dout[lane] = (__bf16)0.f;
  }
  return true;
}

// The candidate pass's merge: one wave per query row (four a workgroup).  A
// row whose regions overflowed, or that holds fewer than min(K, lengths2)
// candidates, joins its cloud's rerun list, as does every row of a cloud
// without the bound (kb_sampled).  Region s's m = a + b candidates
// (the h = 0 half's first a slots, the h = 1 half's last b), in slot order,
// go to lanes 0 .. m - 1 of one register (two when m > 64 for some region).
// NSL: slices rounded up to a multiple of 4.  Rows past lengths1 are (0, 0).
template <int NSL>
__global__ __launch_bounds__(256) void knn_bf16_cmerge_kernel(
    const uint64_t* __restrict__ cand, const int32_t* __restrict__ ccount,
    const int64_t* __restrict__ len1, const int64_t* __restrict__ len2, int64_t rows, int P1,
    int P2, int K, int slices, int64_t* __restrict__ idxs, __bf16* __restrict__ dists,
    int32_t* __restrict__ rlist, int32_t* __restrict__ rcount) {
  static_assert(KB_CAP == 128, "at most two registers a region");
  __shared__ uint32_t s_hist[KB_WAVES][64];
  __shared__ uint64_t s_sel[KB_WAVES][KB_SEL + 64];
  const int w = wave_id(), lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * KB_WAVES + w;
  if (row >= rows) return;
  const int64_t n = row / P1;
  const int pos = (int)(row - n * P1);
  int64_t l1 = len1[n], l2 = len2[n];
  l1 = l1 < 0 ? 0 : (l1 > P1 ? P1 : l1);
  l2 = l2 < 0 ? 0 : (l2 > P2 ? P2 : l2);
  int64_t* __restrict__ io = idxs + row * K;
  __bf16* __restrict__ dout = dists + row * K;
  if (pos >= l1) {
    if (lane < K) {
      io[lane] = 0;
      dout[lane] = (__bf16)0.f;
    }
    return;
  }
  auto rerun = [&]() {
    if (lane == 0) rlist[n * P1 + atomicAdd(&rcount[n], 1)] = pos;
  };
  if (!kb_sampled(l2, K)) {  // a cloud without the bound: no candidates were kept
    rerun();
    return;
  }
  const int32_t* __restrict__ cc = ccount + (size_t)row * slices * 2;
  int ca = 0, cb = 0;
  if (lane < slices) {
    ca = cc[2 * lane];
    cb = cc[2 * lane + 1];
  }
  const bool over = __ballot(ca + cb > KB_CAP) != 0;
  const bool wide = __ballot(ca + cb > 64) != 0;
  const int total = (int)__builtin_amdgcn_readlane((int)kb_wave_scan((uint32_t)(ca + cb)), 63);
  if (over || total < min((int64_t)K, l2)) {
    rerun();
    return;
  }
  const uint64_t* __restrict__ rg = cand + (size_t)row * slices * KB_CAP;
  // element e of region s (e < a + b) lies in slot e (e < a) or e + 128 - a - b
  auto load = [&](int s, int e) __attribute__((always_inline)) {
    const int a = __builtin_amdgcn_readlane(ca, s), b = __builtin_amdgcn_readlane(cb, s);
    return e < a + b ? rg[(size_t)s * KB_CAP + (e < a ? e : e + KB_CAP - a - b)] : ~0ull;
  };
  bool ok;
  if (!wide) {
    uint64_t key[NSL];
#pragma unroll
    for (int s = 0; s < NSL; ++s) key[s] = s < slices ? load(s, lane) : ~0ull;
    ok = kb_select(key, total, K, s_hist[w], s_sel[w], io, dout);
  } else {
    uint64_t key[2 * NSL];
#pragma unroll
    for (int s = 0; s < NSL; ++s) {
      key[2 * s] = s < slices ? load(s, lane) : ~0ull;
      key[2 * s + 1] = s < slices ? load(s, 64 + lane) : ~0ull;
    }
    ok = kb_select(key, total, K, s_hist[w], s_sel[w], io, dout);
  }
  if (!ok) rerun();
}

// Two lanes per query row (lanes j and j + 32 of a wave; 32 rows a wave):
// each merges its half of the row's nl slice lists (sorted keys, K a list,
// padded to KC with the empty key) in registers, v_permlane32_swap gives both
// lanes both halves' lists, and both merge those; lane j writes entries
// [0, KC/2) of the row, lane j + 32 entries [KC/2, KC) (those below K).  Rows
// past lengths1 and empty entries are (0, 0).
// Positions are rows (cloud n, position p: list entry of row n P1 + p), or
// with qlist the rerun list's entries, whose rows are n P1 + qlist[n P1 + p].
template <int KC>
__global__ __launch_bounds__(256) void knn_bf16_merge_kernel(
    const uint64_t* __restrict__ part, const int64_t* __restrict__ len1, int64_t rows, int P1,
    int K, int nl, int64_t* __restrict__ idxs, __bf16* __restrict__ dists,
    const int32_t* __restrict__ qlist, const int32_t* __restrict__ qcount) {
  const int lane = lane_id(), j = lane & 31, h = lane >> 5;
  const int64_t prow = ((int64_t)blockIdx.x * KB_WAVES + wave_id()) * 32 + j;
  const uint64_t empty = kb_key(Lim<float>::inf(), KB_NONE);
  bool real = false;
  int64_t row = prow;  // the output row
  const int64_t n = prow < rows ? prow / P1 : 0;
  const int pos = (int)(prow - n * P1);
  if (prow < rows) {
    if (qlist) {
      real = pos < qcount[n];
      row = real ? n * P1 + qlist[n * P1 + pos] : prow;
    } else {
      int64_t l1 = len1[n];
      l1 = l1 < 0 ? 0 : (l1 > P1 ? P1 : l1);
      real = pos < l1;
    }
  }
  if (qlist && !real && __ballot(real) == 0) return;  // a wave past the rerun list
  uint64_t a[KC];
#pragma unroll
  for (int s = 0; s < KC; ++s) a[s] = empty;
  const int hl = (nl + 1) / 2, L0 = h * hl, L1 = min(nl, L0 + hl);
  if (real && L0 < L1) {
    // entry s of list L: part[((n nl + L) K + s) P1 + q], so the 32 lanes
    // of a half-wave read consecutive keys; the next list is loaded while
    // the current one is merged
    const uint64_t* __restrict__ base = part + (size_t)n * nl * K * P1 + pos;
    auto load = [&](uint64_t (&b)[KC], int L) __attribute__((always_inline)) {
#pragma unroll
      for (int s = 0; s < KC; ++s) b[s] = s < K ? base[((size_t)L * K + s) * P1] : empty;
    };
    load(a, L0);
    uint64_t b[KC];
    if (L0 + 1 < L1) load(b, L0 + 1);
    for (int L = L0 + 1; L < L1; ++L) {
      uint64_t c[KC];
      if (L + 1 < L1) load(c, L + 1);
      kb_merge<KC, KC>(a, b);
#pragma unroll
      for (int s = 0; s < KC; ++s) b[s] = c[s];
    }
  }
  // every lane takes part: lane j's list to lanes j and j + 32 as x, lane
  // j + 32's as y (swap(x, y) leaves x = [x_lo, y_lo], y = [x_hi, y_hi])
  uint64_t x[KC], y[KC];
#pragma unroll
  for (int s = 0; s < KC; ++s) {
    const uint32_t lo = (uint32_t)a[s], hi = (uint32_t)(a[s] >> 32);
    const auto rl = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto rh = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    x[s] = ((uint64_t)rh[0] << 32) | rl[0];
    y[s] = ((uint64_t)rh[1] << 32) | rl[1];
  }
  kb_merge<KC, KC>(x, y);
  if (prow >= rows) return;
  if (qlist && !real) return;
  int64_t* __restrict__ io = idxs + row * K;
  __bf16* __restrict__ dout = dists + row * K;
  const uint32_t upper = bit_mask((uint32_t)h, 0);
#pragma unroll
  for (int s = 0; s < KC / 2; ++s) {
    const int k = s + (h ? KC / 2 : 0);
    const uint32_t kl = vsel_u32(upper, (uint32_t)x[s], (uint32_t)x[s + KC / 2]);
    const uint32_t kh = vsel_u32(upper, (uint32_t)(x[s] >> 32), (uint32_t)(x[s + KC / 2] >> 32));
    if (k < K) {
      const bool ok = real && kl != (uint32_t)KB_NONE;  // fewer than K references
      io[k] = ok ? (int64_t)kl : 0;
      dout[k] = ok ? (__bf16)__uint_as_float(kh) : (__bf16)0.f;
    }
  }
}

static int64_t kb_align(int64_t x) { return (x + 255) / 256 * 256; }


// Workspace: norms (float per point, rows padded to 32), the partial lists,
// then (sampled bound) its parts (KB_TP x KB_TK floats per query), the rerun
// counts (int32 per cloud), the rerun lists (int32 per query), the candidate
// regions (KB_CAP keys per query and candidate slice) and their counts (two
// int32 per query and candidate slice).
struct KbWs {
  int64_t part, taup, rcount, rlist, cand, ccount, total;
};
static KbWs kb_ws(int64_t N, int64_t P1, int64_t P2, int64_t K) {
  const KbPlan p = kb_plan(N, P1, P2);
  KbWs w;
  w.part = kb_align(N * (kb_pad(P1) + kb_pad(P2)) * 4);
  int64_t o = w.part + kb_align(N * P1 * p.slices * K * 8);
  w.taup = w.rcount = w.rlist = w.cand = w.ccount = -1;
  if (kb_sampled(P2, K)) {
    const int64_t cs = kb_cplan(N, P1, P2).slices;
    w.taup = o;
    o += kb_align(N * P1 * KB_TP * KB_TK * 4);
    w.rcount = o;
    o += kb_align(N * 4);
    w.rlist = o;
    o += kb_align(N * P1 * 4);
    w.cand = o;
    o += kb_align(N * P1 * cs * KB_CAP * 8);
    w.ccount = o;
    o += kb_align(N * P1 * cs * 2 * 4);
  }
  w.total = o;
  return w;
}

int64_t knn_bf16_workspace(int64_t N, int64_t P1, int64_t P2, int64_t K) {
  return kb_ws(N, P1, P2, K).total;
}

bool knn_bf16_supported(int64_t D, int64_t K, int norm) {
  return norm == 2 && D % 8 == 0 && D >= 8 && D <= KB_DMAX && K >= 1 && K <= 32;
}

struct KbArgs {
  const __bf16 *p1, *p2;
  const int64_t *l1, *l2;
  int N, P1, P2, D, K;
  const float *qn, *rn;
  uint64_t* part;
  float* taup;  // null: no sampled bound
  int32_t *rlist, *rcount;
  uint64_t* cand;
  int32_t* ccount;
  int64_t* idxs;
  __bf16* dists;
  hipStream_t s;
};

// Sampled bound (when it applies): its parts, the candidate pass under it
// and its merge (which lists the rows it cannot settle), then the exact pass
// -- slices with lists, and their merge -- over those rows only.  Without the
// bound, the exact pass over every row.
template <int KS, bool HALF, int KC>
static void kb_launch(const KbArgs& a) {
  const KbPlan p = kb_plan(a.N, a.P1, a.P2);
  const dim3 grid(a.N * p.nqb * p.slices), blk(256);
  const int64_t r1 = (int64_t)a.N * a.P1;
  const dim3 mg((unsigned)((r1 + 32 * KB_WAVES - 1) / (32 * KB_WAVES))), mb(64 * KB_WAVES);
  if (!a.taup) {
    hipLaunchKernelGGL((knn_bf16_slice_kernel<KS, HALF, KC>), grid, blk, 0, a.s, a.p1, a.p2, a.l1,
                       a.l2, a.P1, a.P2, a.D, a.K, p.nqb, p.slices, a.qn, a.rn, a.part,
                       (const int32_t*)nullptr, (const int32_t*)nullptr);
    hipLaunchKernelGGL(knn_bf16_merge_kernel<KC>, mg, mb, 0, a.s, (const uint64_t*)a.part, a.l1,
                       r1, a.P1, a.K, p.slices, a.idxs, a.dists, (const int32_t*)nullptr,
                       (const int32_t*)nullptr);
    return;
  }
  const KbPlan cp = kb_cplan(a.N, a.P1, a.P2);
  hipLaunchKernelGGL((knn_bf16_tau_kernel<KS, HALF>), dim3(a.N * p.nqb * KB_TP), blk, 0, a.s,
                     a.p1, a.p2, a.l1, a.l2, a.N, a.P1, a.P2, a.K, p.nqb, a.qn, a.rn, a.taup,
                     a.rcount);
  hipLaunchKernelGGL((knn_bf16_cand_kernel<KS, HALF>), dim3(a.N * cp.nqb * cp.slices), blk, 0, a.s,
                     a.p1, a.p2, a.l1, a.l2, a.P1, a.P2, a.K, cp.nqb, cp.slices, a.qn, a.rn,
                     (const float*)a.taup, a.cand, a.ccount);
  {
    const dim3 g((unsigned)((r1 + KB_WAVES - 1) / KB_WAVES));
#define KB_CM(NSL)                                                                               \
  hipLaunchKernelGGL(knn_bf16_cmerge_kernel<NSL>, g, blk, 0, a.s, (const uint64_t*)a.cand,       \
                     (const int32_t*)a.ccount, a.l1, a.l2, r1, a.P1, a.P2, a.K, cp.slices, a.idxs, \
                     a.dists, a.rlist, a.rcount)
    if (cp.slices <= 4) KB_CM(4);
    else if (cp.slices <= 8) KB_CM(8);
    else if (cp.slices <= 12) KB_CM(12);
    else KB_CM(16);
#undef KB_CM
  }
  hipLaunchKernelGGL((knn_bf16_slice_kernel<KS, HALF, KC>), grid, blk, 0, a.s, a.p1, a.p2, a.l1,
                     a.l2, a.P1, a.P2, a.D, a.K, p.nqb, p.slices, a.qn, a.rn, a.part,
                     (const int32_t*)a.rlist, (const int32_t*)a.rcount);
  hipLaunchKernelGGL(knn_bf16_merge_kernel<KC>, mg, mb, 0, a.s, (const uint64_t*)a.part, a.l1,
                     r1, a.P1, a.K, p.slices, a.idxs, a.dists, (const int32_t*)a.rlist,
                     (const int32_t*)a.rcount);
}

template <int KC>
static void kb_dispatch_ks(const KbArgs& a) {
  // D % 8 == 0, 8 <= D <= 128: D / 8 = 2 KS - HALF
#define KB_CASE(DD, KS_, HALF_) \
  case DD: kb_launch<KS_, HALF_, KC>(a); break;
  switch (a.D) {
    KB_CASE(8, 1, true) KB_CASE(16, 1, false) KB_CASE(24, 2, true) KB_CASE(32, 2, false)
    KB_CASE(40, 3, true) KB_CASE(48, 3, false) KB_CASE(56, 4, true) KB_CASE(64, 4, false)
    KB_CASE(72, 5, true) KB_CASE(80, 5, false) KB_CASE(88, 6, true) KB_CASE(96, 6, false)
    KB_CASE(104, 7, true) KB_CASE(112, 7, false) KB_CASE(120, 8, true)
    default: kb_launch<8, false, KC>(a); break;
  }
#undef KB_CASE
}

void launch_knn_bf16(const void* p1, const void* p2, const int64_t* l1, const int64_t* l2, int N,
                     int P1, int P2, int D, int K, int64_t* idxs, void* dists, void* ws,
                     hipStream_t s) {
  const KbWs L = kb_ws(N, P1, P2, K);
  char* wb = reinterpret_cast<char*>(ws);
  float* qn = reinterpret_cast<float*>(ws);
  float* rn = qn + (size_t)N * kb_pad(P1);
  const int64_t r1 = (int64_t)N * P1, r2 = (int64_t)N * P2;
  const int64_t nb1 = (r1 + 15) / 16, nb2 = (r2 + 15) / 16;
  if (nb1 + nb2 > 0)
    hipLaunchKernelGGL(knn_bf16_norms_kernel, dim3((unsigned)(nb1 + nb2)), dim3(256), 0, s,
                       (const __bf16*)p1, r1, (int64_t)P1, qn, (const __bf16*)p2, r2, (int64_t)P2,
                       rn, D, nb1);
  if (r1 == 0) return;
  KbArgs a;
  a.p1 = (const __bf16*)p1;
  a.p2 = (const __bf16*)p2;
  a.l1 = l1;
  a.l2 = l2;
  a.N = N;
  a.P1 = P1;
  a.P2 = P2;
  a.D = D;
  a.K = K;
  a.qn = qn;
  a.rn = rn;
  a.part = reinterpret_cast<uint64_t*>(wb + L.part);
  a.taup = L.taup >= 0 ? reinterpret_cast<float*>(wb + L.taup) : nullptr;
  a.rcount = L.rcount >= 0 ? reinterpret_cast<int32_t*>(wb + L.rcount) : nullptr;
  a.rlist = L.rlist >= 0 ? reinterpret_cast<int32_t*>(wb + L.rlist) : nullptr;
  a.cand = L.cand >= 0 ? reinterpret_cast<uint64_t*>(wb + L.cand) : nullptr;
  a.ccount = L.ccount >= 0 ? reinterpret_cast<int32_t*>(wb + L.ccount) : nullptr;
  a.idxs = idxs;
  a.dists = (__bf16*)dists;
  a.s = s;
  if (K <= 16) kb_dispatch_ks<16>(a);
  else kb_dispatch_ks<32>(a);
}

}  // namespace tpo
