// chamfer_dense.hpp -- the brute-force Chamfer forward for one block of
// 64*Q queries of one (cloud, direction), shared by chamfer.hip's dense
// kernels and the grid search (which runs it for clouds whose grid is
// degenerate).  Both follow the reference's first-index rule
// (chamfer.cu:69-72, 159-162): the block's 4 waves split the other cloud into
// 4 chunks whose results merge in index order with strict-less.
#pragma once
#include "chamfer_common.hpp"

#pragma clang fp contract(off)

namespace tpo {

// Copy a wave-uniform (SGPR) value into a VGPR.  On gfx950 a VALU op with an
// SGPR source issues at 4 cycles per wave64 instruction, while VGPR-only
// FP32 ops issue at ~2.3-2.7; one v_mov per reference coordinate, shared by
// the Q queries of the lane, lets every subtraction use VGPR operands.  The
// empty asm only pins the value to a VGPR: the compiler emits the move (and
// any wait it needs) itself.
__device__ __forceinline__ float to_vgpr(float s) {
  float v = s;
  asm("" : "+v"(v));
  return v;
}
__device__ __forceinline__ double to_vgpr(double s) { return s; }
__device__ __forceinline__ half_t to_vgpr(half_t s) { return s; }

__device__ __forceinline__ float vmin(float a, float b) { return __builtin_fminf(a, b); }
__device__ __forceinline__ double vmin(double a, double b) { return __builtin_fmin(a, b); }
__device__ __forceinline__ half_t vmin(half_t a, half_t b) { return __builtin_fminf16(a, b); }

// Reference formula per pair (double / half, and float without a workspace
// below the filter's sizes): keeps per-tile minima and re-scans the winning
// tile for the first index.  qp / rp: the query and reference clouds; dout /
// iout: the query cloud's outputs; queries qb*64*Q + [0, 64*Q).
template <typename T, int Q>
__device__ __forceinline__ void chamfer_dense_block(const T* __restrict__ qp,
                                                    const T* __restrict__ rp, int nq, int nr,
                                                    int qb, T* __restrict__ dout,
                                                    int32_t* __restrict__ iout,
                                                    T (&s_d)[CH_WAVES][64 * Q],
                                                    int (&s_i)[CH_WAVES][64 * Q]) {
  const int w = wave_id(), lane = lane_id();
  const int chunk = ((nr + CH_WAVES * CH_TILE - 1) / (CH_WAVES * CH_TILE)) * CH_TILE;
  const int c0 = w * chunk;
  const int c1 = min(nr, c0 + chunk);

  T qx[Q], qy[Q], qz[Q], best[Q];
  int bt[Q];
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    int gq = qb * 64 * Q + i * 64 + lane;
    gq = gq < nq ? gq : nq - 1;
    qx[i] = qp[3 * gq];
    qy[i] = qp[3 * gq + 1];
    qz[i] = qp[3 * gq + 2];
    best[i] = Lim<T>::inf();
    bt[i] = c0;
  }

  int t0 = c0;
  for (; t0 + CH_TILE <= c1; t0 += CH_TILE) {
    T tmin[Q];
#pragma unroll
    for (int i = 0; i < Q; ++i) tmin[i] = Lim<T>::inf();
    const T* __restrict__ r = rp + 3 * t0;
#pragma unroll
    for (int j = 0; j < CH_TILE; ++j) {
      const T rx = to_vgpr(r[3 * j]), ry = to_vgpr(r[3 * j + 1]), rz = to_vgpr(r[3 * j + 2]);
#pragma unroll
      for (int i = 0; i < Q; ++i)
        tmin[i] = vmin(tmin[i], sq3((T)(rx - qx[i]), (T)(ry - qy[i]), (T)(rz - qz[i])));
    }
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const bool lt = tmin[i] < best[i];
      best[i] = lt ? tmin[i] : best[i];
      bt[i] = lt ? t0 : bt[i];
    }
  }
  if (t0 < c1) {  // partial last tile of this chunk
    T tmin[Q];
#pragma unroll
    for (int i = 0; i < Q; ++i) tmin[i] = Lim<T>::inf();
    for (int j = t0; j < c1; ++j) {
      const T rx = rp[3 * j], ry = rp[3 * j + 1], rz = rp[3 * j + 2];
#pragma unroll
      for (int i = 0; i < Q; ++i)
        tmin[i] = vmin(tmin[i], sq3((T)(rx - qx[i]), (T)(ry - qy[i]), (T)(rz - qz[i])));
    }
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const bool lt = tmin[i] < best[i];
      best[i] = lt ? tmin[i] : best[i];
      bt[i] = lt ? t0 : bt[i];
    }
  }

  // With finite coordinates no distance is NaN (overflow gives +inf), so the
  // first index of the minimum is the reference's answer: recover it inside
  // the winning tile (same formula, same bits).  Non-finite coordinates in
  // the chunk (or its first 512-stage head) or the query: chunk_scan.
  bool rfin = true;
  for (int j = c0 + lane; j < c1; j += 64) rfin = rfin && finite3(rp + 3 * j);
  if (c0 < c1 && (c0 & 511) != 0) rfin = rfin && finite3(rp + 3 * (c0 & ~511));
  const bool rbad = __ballot(!rfin) != 0;
  int found[Q];
  uint64_t amb[Q];
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    int gq = qb * 64 * Q + i * 64 + lane;
    gq = gq < nq ? gq : nq - 1;
    const bool a = c0 < c1 && (rbad || !finite3(qp + 3 * gq));
    amb[i] = __ballot(a);
    found[i] = 0x7fffffff;
    if (c0 < c1 && !a) {
      const int tb = bt[i];
      const int te = min(tb + CH_TILE, c1);
      for (int j = tb; j < te; ++j) {
        if (ref_d(qx[i], qy[i], qz[i], rp + 3 * j) == best[i]) {
          found[i] = j;
          break;
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    uint64_t m = amb[i];
    while (m) {
      const int l = __builtin_ctzll(m);
      m &= m - 1;
      int gq = qb * 64 * Q + i * 64 + l;
      gq = gq < nq ? gq : nq - 1;
      T md;
      int mi;
      chunk_scan(qp[3 * gq], qp[3 * gq + 1], qp[3 * gq + 2], rp, c0, c1, lane, md, mi);
      if (lane == l) {
        best[i] = md;
        found[i] = mi;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    s_d[w][i * 64 + lane] = best[i];
    s_i[w][i * 64 + lane] = found[i];
  }
  __syncthreads();

  for (int e = threadIdx.x; e < 64 * Q; e += 256) {
    const int gq = qb * 64 * Q + e;
    if (gq >= nq) continue;
    T bd;
    int bi;
    merge_chunks<T, 64 * Q>(&s_d[0][e], &s_i[0][e], bd, bi);
    dout[gq] = bd;
    iout[gq] = bi;
  }
}

// ------------------------------------------------- forward, float: filter
// Expanded-form filter (float).  For query q and reference r
//   A(r) = |r|^2 - 2 q.r = fma(-2qx, rx, fma(-2qy, ry, fma(-2qz, rz, |r|^2)))
// costs 3 FMAs per pair instead of the reference formula's 6 VALU ops.  With
// u = 2^-24 and every coordinate below 2^60 in magnitude (so nothing
// overflows), A(r) differs from D(r) - |q|^2, D being the reference formula's
// float result, by at most
//   E(r) <= 6u(|r|^2 + |q||r|) + 5u D(r) <= 21u|q|^2 + 20u D(r)
// (four roundings in A; the reference formula's relative error is <= 5u since
// all its terms are non-negative; |r| <= |q| + sqrt(D)).  Per tile of 16
// references the kernel keeps the tile minimum of A, per query the best tile
// (strictly smaller replaces, so the earliest wins) and `second`, the
// minimum over every other tile.  With a* the best value and
//   W = 2^-18 (|q|^2 + max(a* + |q|^2, 0)) + 2^-120,
// W >= E(r*) + E(ra) for an exact minimiser r* and the approximate one ra
// (the 2^-120 term covers gradual underflow), so A(r*) <= a* + W.  Hence if
// second > a* + W every exact minimiser lies in the best tile, which is
// re-scanned with the reference formula: same bits, first index.  Otherwise
// (a near-tie across tiles, NaN/Inf or a coordinate >= 2^60 in the wave's
// chunk or the query, an empty chunk) the whole wave re-scans that query's
// chunk with the reference formula, lanes striding the references.
//   The references reach the lanes through a wave-private LDS block: each
// lane loads one reference and computes |r|^2 once, and every pair then
// reads it back as one broadcast ds_read_b128, so the per-pair VALU work is
// the 3 FMAs, half a v_min3 and the per-tile bookkeeping.
constexpr int CH_FTILE = 16;  // references per tile of the filter kernel

template <int Q, int TT>
__device__ __forceinline__ void chamfer_filter_block(const float* __restrict__ qp,
                                                     const float* __restrict__ rp, int nq, int nr,
                                                     int qb, float* __restrict__ dout,
                                                     int32_t* __restrict__ iout,
                                                     float4 (&s_ref)[CH_WAVES][64],
                                                     float (&s_d)[CH_WAVES][64 * Q],
                                                     int (&s_i)[CH_WAVES][64 * Q]) {
  const int w = wave_id(), lane = lane_id();
  const int chunk = ((nr + CH_WAVES * 64 - 1) / (CH_WAVES * 64)) * 64;
  const int c0 = min(nr, w * chunk);
  const int c1 = min(nr, c0 + chunk);

  float bd[Q];
  int bi[Q];
  if (c0 < c1) {
    float qx2[Q], qy2[Q], qz2[Q], best[Q], second[Q];
    int bt[Q];
    uint32_t qbig = 0;  // bit i: query i has a non-finite or >= 2^60 coordinate
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      int gq = qb * 64 * Q + i * 64 + lane;
      gq = gq < nq ? gq : nq - 1;
      const float x = qp[3 * gq], y = qp[3 * gq + 1], z = qp[3 * gq + 2];
      qx2[i] = -2.f * x;
      qy2[i] = -2.f * y;
      qz2[i] = -2.f * z;
      if (max(abs_bits(x), max(abs_bits(y), abs_bits(z))) >= CH_BIG) qbig |= 1u << i;
      best[i] = Lim<float>::inf();
      second[i] = Lim<float>::inf();
      bt[i] = c0;
    }
    uint32_t rbig = 0;
    float nx, ny, nz;
    {
      const int j = min(c0 + lane, c1 - 1);
      nx = rp[3 * j];
      ny = rp[3 * j + 1];
      nz = rp[3 * j + 2];
    }
    for (int blk = c0; blk < c1; blk += 64) {
      const float x = nx, y = ny, z = nz;
      rbig = max(rbig, max(abs_bits(x), max(abs_bits(y), abs_bits(z))));
      // references past the chunk: A = +inf, never a tile minimum
      const float rr = blk + lane < c1 ? sq3(x, y, z) : Lim<float>::inf();
      s_ref[w][lane] = make_float4(x, y, z, rr);
      __builtin_amdgcn_wave_barrier();
      const int jn = min(blk + 64 + lane, c1 - 1);  // unconditional prefetch
      nx = rp[3 * jn];
      ny = rp[3 * jn + 1];
      nz = rp[3 * jn + 2];
#pragma unroll
      for (int t = 0; t < 64 / TT; ++t) {
        float tmin[Q];
#pragma unroll
        for (int jj = 0; jj < TT; ++jj) {
          const float4 r = s_ref[w][TT * t + jj];
#pragma unroll
          for (int i = 0; i < Q; ++i) {
            const float a = __builtin_fmaf(qx2[i], r.x,
                                           __builtin_fmaf(qy2[i], r.y, __builtin_fmaf(qz2[i], r.z, r.w)));
            tmin[i] = jj == 0 ? a : fminf(tmin[i], a);
          }
        }
        const int t0 = blk + TT * t;
#pragma unroll
        for (int i = 0; i < Q; ++i) {
          const bool lt = tmin[i] < best[i];
          second[i] = lt ? best[i] : fminf(second[i], tmin[i]);
          best[i] = lt ? tmin[i] : best[i];
          bt[i] = lt ? t0 : bt[i];
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
    // the 512-stage head of c0 decides whether the chunk's first references
    // count (NaN rule of chunk_scan), so it joins the check
    if ((c0 & 511) != 0) {
      const float* h = rp + 3 * (c0 & ~511);
      rbig = max(rbig, max(abs_bits(h[0]), max(abs_bits(h[1]), abs_bits(h[2]))));
    }
    const bool rbad = __ballot(rbig >= CH_BIG) != 0;

    uint64_t amb[Q];
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const float qq = 0.25f * sq3(qx2[i], qy2[i], qz2[i]);
      const float W = __builtin_fmaf(0x1p-18f, qq + fmaxf(best[i] + qq, 0.f), 0x1p-120f);
      const bool a = rbad || ((qbig >> i) & 1u) || !(second[i] > best[i] + W);
      amb[i] = __ballot(a);
      float d_ = Lim<float>::inf();
      int i_ = 0x7fffffff;
      if (!a) {  // all exact minimisers are in tile bt: first index of its minimum
        const float x = -0.5f * qx2[i], y = -0.5f * qy2[i], z = -0.5f * qz2[i];
        const int te = min(bt[i] + TT, c1);
        for (int j = bt[i]; j < te; ++j) {
          const float d = ref_d(x, y, z, rp + 3 * j);
          if (d < d_) {
            d_ = d;
            i_ = j;
          }
        }
      }
      bd[i] = d_;
      bi[i] = i_;
    }
    // ambiguous queries: the wave scans the chunk for one query at a time
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      uint64_t m = amb[i];
      while (m) {
        const int l = __builtin_ctzll(m);
        m &= m - 1;
        int gq = qb * 64 * Q + i * 64 + l;
        gq = gq < nq ? gq : nq - 1;
        float md;
        int mi;
        chunk_scan(qp[3 * gq], qp[3 * gq + 1], qp[3 * gq + 2], rp, c0, c1, lane, md, mi);
        if (lane == l) {
          bd[i] = md;
          bi[i] = mi;
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      bd[i] = Lim<float>::inf();
      bi[i] = 0x7fffffff;
    }
  }
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    s_d[w][i * 64 + lane] = bd[i];
    s_i[w][i * 64 + lane] = bi[i];
  }
  __syncthreads();

  for (int e = threadIdx.x; e < 64 * Q; e += 256) {
    const int gq = qb * 64 * Q + e;
    if (gq >= nq) continue;
    float d;
    int ix;
    merge_chunks<float, 64 * Q>(&s_d[0][e], &s_i[0][e], d, ix);
    dout[gq] = d;
    iout[gq] = ix;
  }
}

}  // namespace tpo
