/*
 * tpo_oracle.c -- CPU restatement of the reference's nearest-neighbour path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the thing measured or
 * shipped).  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg load this library.
 *
 * Reference files restated (paths relative to the reference repository):
 *   torch_point_ops/chamfer/csrc/cuda/chamfer.cu   chamfer forward/backward
 *   torch_point_ops/knn/csrc/cuda/knn.cu           KNN kernels V0..V3, backward
 *   torch_point_ops/knn/csrc/cuda/utils/mink.cuh   MinK / RegisterMinK
 *   torch_point_ops/knn/csrc/cuda/utils/dispatch.cuh  version selection
 *   torch_point_ops/fps/csrc/cuda/fps.cu           FPS kernel, gather kernels
 *   torch_point_ops/knn/csrc/knn.cpp, fps/csrc/fps.cpp   CPU kernels (baseline)
 *
 * Arithmetic model.  Values of every dtype are carried in a C double (exact
 * for binary16/binary32 values) and every operation rounds to the dtype:
 *   float32  each + - * is done in C float (SSE, no excess precision);
 *   float64  in double;
 *   float16  in float, then rounded to binary16 -- c10::Half's operators
 *            (torch/headeronly/util/Half.h) convert both operands to float,
 *            operate, and convert the float result back with RNE.
 * The reference's CUDA build runs nvcc with its default -fmad=true
 * (setup.py:83-92), which contracts the distance sums.  Contraction cannot be
 * observed here (no nvcc), so the oracle pins the order LLVM/NVPTX forms from
 * the source expressions:
 *   chamfer.cu:67 / fps.cu:142,145   x*x + y*y + z*z  ->  fma(z,z, fma(x,x, y*y))
 *   knn.cu:149-158 (dist += diff*diff over d)          ->  fma(d2,d2, fma(d1,d1, d0*d0))
 * This file must be built with -ffp-contract=off so gcc adds no contraction
 * of its own; the explicit fma()/fmaf() calls are the only fused operations.
 */
#include "tpo_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define INLINE static inline __attribute__((always_inline))

/* ------------------------------------------------------------------ */
/* binary16 / bfloat16 conversions                                     */
/* ------------------------------------------------------------------ */

uint16_t tpo_ref_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) {                 /* inf / nan */
    return (uint16_t)(sign | (ax == 0x7f800000u ? 0x7c00u : 0x7e00u));
  }
  int32_t e = (int32_t)(ax >> 23) - 127;   /* unbiased exponent */
  uint32_t m = ax & 0x7fffffu;
  if (e > 15) return (uint16_t)(sign | 0x7c00u);  /* overflow -> inf */
  if (e >= -14) {                          /* normal half (may round up) */
    uint32_t h = ((uint32_t)(e + 15) << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* carry ok */
    return (uint16_t)(sign | h);
  }
  if ((ax >> 23) == 0) return sign;        /* float subnormal or zero */
  /* half subnormal: value = M * 2^(e-23), unit 2^-24 -> M >> s, s = -e-1 */
  uint32_t M = m | 0x800000u;
  int32_t s = -e - 1;                      /* s >= 14 */
  if (s > 24) return sign;                 /* < 2^-25 -> 0 */
  uint32_t h = M >> s;
  uint32_t rem = M & ((1u << s) - 1u);
  uint32_t half = 1u << (s - 1);
  if (rem > half || (rem == half && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

float tpo_ref_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  float out;
  if (e == 0x1f) {
    uint32_t x = sign | 0x7f800000u | (m << 13);
    memcpy(&out, &x, 4);
    return out;
  }
  if (e == 0) {
    out = ldexpf((float)m, -24);
    return sign ? -out : out;
  }
  uint32_t x = sign | ((e + 112u) << 23) | (m << 13);
  memcpy(&out, &x, 4);
  return out;
}

uint16_t tpo_ref_f32_to_bf16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

float tpo_ref_bf16_to_f32(uint16_t h) {
  uint32_t x = (uint32_t)h << 16;
  float out;
  memcpy(&out, &x, 4);
  return out;
}

void tpo_ref_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = tpo_ref_f32_to_f16(in[i]);
}
void tpo_ref_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = tpo_ref_f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------ */
/* dtype-generic arithmetic (dt is a literal at every call site, so the */
/* switches fold away after inlining)                                   */
/* ------------------------------------------------------------------ */

/* A float rounded to the nearest binary16 value (ties to even), returned as a
   float, without the round trip through the 16-bit encoding:
   - |v| >= 2^-14 (normal halves): the 23-bit significand is rounded to 10
     bits (add 0xfff plus the lowest kept bit, which breaks ties to even,
     then clear the 13 dropped bits; a carry moves into the exponent as it
     should); a result of 2^16 or more (from 65520 up) is infinite;
   - |v| < 2^-14: halves there are the multiples of 2^-24, so the result is
     |v| 2^24 rounded to an integer (adding and subtracting 2^23 in float
     rounds a value below 2^23 to the nearest integer, ties to even), times
     2^-24; both scalings are exact;
   - NaN becomes the quiet NaN 0x7e00 and infinities stay, signs kept, as
     tpo_ref_f32_to_f16 encodes them.
   tpo_ref_f16_round_check compares it with tpo_ref_f16_to_f32 of
   tpo_ref_f32_to_f16 over every float bit pattern. */
INLINE float rh_float(float v) {
  uint32_t x, r;
  memcpy(&x, &v, 4);
  const uint32_t sign = x & 0x80000000u, ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) {
    r = ax == 0x7f800000u ? 0x7f800000u : 0x7fc00000u;
  } else if (ax >= 0x38800000u) {
    r = (ax + 0xfffu + ((ax >> 13) & 1u)) & 0xffffe000u;
    if (r >= 0x47800000u) r = 0x7f800000u;
  } else {
    float a;
    memcpy(&a, &ax, 4);
    const float y = a * 0x1p24f;
    const float q = ((y + 0x1p23f) - 0x1p23f) * 0x1p-24f;
    memcpy(&r, &q, 4);
  }
  r |= sign;
  float out;
  memcpy(&out, &r, 4);
  return out;
}

int64_t tpo_ref_f16_round_check(void) {
  int64_t bad = 0;
#ifdef _OPENMP
#pragma omp parallel for reduction(+ : bad) schedule(static)
#endif
  for (int64_t i = 0; i < ((int64_t)1 << 32); ++i) {
    const uint32_t x = (uint32_t)i;
    float f;
    memcpy(&f, &x, 4);
    const float a = rh_float(f), b = tpo_ref_f16_to_f32(tpo_ref_f32_to_f16(f));
    uint32_t ua, ub;
    memcpy(&ua, &a, 4);
    memcpy(&ub, &b, 4);
    bad += ua != ub;
  }
  return bad;
}

INLINE double rh(float v) { return (double)rh_float(v); }

INLINE double ld(int dt, const void* p, int64_t i) {
  switch (dt) {
    case TPO_REF_F32: return (double)((const float*)p)[i];
    case TPO_REF_F64: return ((const double*)p)[i];
    case TPO_REF_F16: return (double)tpo_ref_f16_to_f32(((const uint16_t*)p)[i]);
    default: return (double)tpo_ref_bf16_to_f32(((const uint16_t*)p)[i]);
  }
}
/* v must already be a value of the dtype (all stores here are). */
INLINE void st(int dt, void* p, int64_t i, double v) {
  switch (dt) {
    case TPO_REF_F32: ((float*)p)[i] = (float)v; break;
    case TPO_REF_F64: ((double*)p)[i] = v; break;
    case TPO_REF_F16: ((uint16_t*)p)[i] = tpo_ref_f32_to_f16((float)v); break;
    default: ((uint16_t*)p)[i] = tpo_ref_f32_to_bf16((float)v); break;
  }
}
/* round an arbitrary double to the dtype (used once, after f64 accumulation) */
INLINE double rnd(int dt, double v) {
  switch (dt) {
    case TPO_REF_F32: return (double)(float)v;
    case TPO_REF_F64: return v;
    case TPO_REF_F16: return rh((float)v);
    default: return (double)tpo_ref_bf16_to_f32(tpo_ref_f32_to_bf16((float)v));
  }
}
INLINE double op_sub(int dt, double a, double b) {
  switch (dt) {
    case TPO_REF_F64: return a - b;
    case TPO_REF_F16: return rh((float)a - (float)b);
    default: return (double)((float)a - (float)b);
  }
}
INLINE double op_add(int dt, double a, double b) {
  switch (dt) {
    case TPO_REF_F64: return a + b;
    case TPO_REF_F16: return rh((float)a + (float)b);
    default: return (double)((float)a + (float)b);
  }
}
INLINE double op_mul(int dt, double a, double b) {
  switch (dt) {
    case TPO_REF_F64: return a * b;
    case TPO_REF_F16: return rh((float)a * (float)b);
    default: return (double)((float)a * (float)b);
  }
}
INLINE double op_fma(int dt, double a, double b, double c) {
  switch (dt) {
    case TPO_REF_F64: return fma(a, b, c);
    default: return (double)fmaf((float)a, (float)b, (float)c);
  }
}

/* Squared distance of chamfer.cu:64-67 and fps.cu:142,145:
   x*x + y*y + z*z.  f32/f64: fma(z,z, fma(x,x, y*y)).
   f16: ((x*x + y*y) + z*z) rounded after every operation. */
INLINE double sq3(int dt, double x, double y, double z) {
  if (dt == TPO_REF_F16) {
    return op_add(dt, op_add(dt, op_mul(dt, x, x), op_mul(dt, y, y)), op_mul(dt, z, z));
  }
  return op_fma(dt, z, z, op_fma(dt, x, x, op_mul(dt, y, y)));
}

/* ------------------------------------------------------------------ */
/* Chamfer                                                             */
/* ------------------------------------------------------------------ */

/* chamfer.cu:36-167: refs staged in tiles of 512; inside a tile the first
   element is taken unconditionally and later ones replace on strict less
   (:69-72); a tile's result replaces the stored one when it is the first tile
   or the stored distance is strictly greater (:159-162).  Outputs start at
   zero (chamfer.cu:176-181), so m == 0 leaves dist = 0, idx = 0. */
INLINE void chamfer_dir(int dt, const void* q, const void* r, int64_t B,
                        int64_t n, int64_t m, void* dist, int32_t* idx) {
  const int64_t tile = 512;
  /* every (cloud, query) is independent: threads change nothing but speed */
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(dynamic, 64)
#endif
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t j = 0; j < n; ++j) {
      const int64_t qi = (b * n + j) * 3;
      const double x1 = ld(dt, q, qi), y1 = ld(dt, q, qi + 1), z1 = ld(dt, q, qi + 2);
      double stored = 0.0;
      int32_t stored_i = 0;
      for (int64_t k2 = 0; k2 < m; k2 += tile) {
        const int64_t end_k = (m < k2 + tile ? m : k2 + tile) - k2;
        double best = 0.0;
        int32_t besti = 0;
        for (int64_t k = 0; k < end_k; ++k) {
          const int64_t ri = (b * m + k2 + k) * 3;
          const double x2 = op_sub(dt, ld(dt, r, ri), x1);
          const double y2 = op_sub(dt, ld(dt, r, ri + 1), y1);
          const double z2 = op_sub(dt, ld(dt, r, ri + 2), z1);
          const double d = sq3(dt, x2, y2, z2);
          if (k == 0 || d < best) {
            best = d;
            besti = (int32_t)(k + k2);
          }
        }
        if (k2 == 0 || stored > best) {
          stored = best;
          stored_i = besti;
        }
      }
      st(dt, dist, b * n + j, stored);
      idx[b * n + j] = stored_i;
    }
  }
}

static int chamfer_fwd_dt(int dt, const void* xyz1, const void* xyz2, int64_t B,
                          int64_t N, int64_t M, void* d1, void* d2, int32_t* i1,
                          int32_t* i2) {
  chamfer_dir(dt, xyz1, xyz2, B, N, M, d1, i1);
  chamfer_dir(dt, xyz2, xyz1, B, M, N, d2, i2);
  return 0;
}

int tpo_ref_chamfer_fwd(int dtype, const void* xyz1, const void* xyz2, int64_t B,
                        int64_t N, int64_t M, void* dist1, void* dist2,
                        int32_t* idx1, int32_t* idx2) {
  if (B < 0 || N < 0 || M < 0) return -1;
  switch (dtype) {
    case TPO_REF_F32: return chamfer_fwd_dt(TPO_REF_F32, xyz1, xyz2, B, N, M, dist1, dist2, idx1, idx2);
    case TPO_REF_F64: return chamfer_fwd_dt(TPO_REF_F64, xyz1, xyz2, B, N, M, dist1, dist2, idx1, idx2);
    case TPO_REF_F16: return chamfer_fwd_dt(TPO_REF_F16, xyz1, xyz2, B, N, M, dist1, dist2, idx1, idx2);
    default: return -2;
  }
}

/* chamfer.cu:200-234 for one direction: g = grad*2 (in dtype, :222);
   c = g*(q - r); grad_q[j] += c; grad_r[idx[j]] += -c (:226-231).
   Contributions go either straight into the dtype outputs (sequential order)
   or into double accumulators. */
INLINE void chamfer_bwd_dir(int dt, const void* q, const void* r, const int32_t* idx,
                            const void* gd, int64_t B, int64_t n, int64_t m,
                            void* gq, void* gr, double* aq, double* ar) {
  if (m == 0) return; /* idx would address an empty cloud */
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t j = 0; j < n; ++j) {
      const int64_t j2 = idx[b * n + j];
      if (j2 < 0 || j2 >= m) continue;
      const double g = op_mul(dt, ld(dt, gd, b * n + j), 2.0);
      for (int c = 0; c < 3; ++c) {
        const int64_t qi = (b * n + j) * 3 + c, ri = (b * m + j2) * 3 + c;
        const double v = op_mul(dt, g, op_sub(dt, ld(dt, q, qi), ld(dt, r, ri)));
        if (aq) {
          aq[qi] += v;
          ar[ri] -= v;
        } else {
          st(dt, gq, qi, op_add(dt, ld(dt, gq, qi), v));
          st(dt, gr, ri, op_add(dt, ld(dt, gr, ri), -v));
        }
      }
    }
  }
}

static int chamfer_bwd_dt(int dt, const void* xyz1, const void* xyz2, const int32_t* idx1,
                          const int32_t* idx2, const void* gd1, const void* gd2, int64_t B,
                          int64_t N, int64_t M, void* g1, void* g2, int accum_f64) {
  for (int64_t i = 0; i < B * N * 3; ++i) st(dt, g1, i, 0.0);
  for (int64_t i = 0; i < B * M * 3; ++i) st(dt, g2, i, 0.0);
  if (!accum_f64) {
    chamfer_bwd_dir(dt, xyz1, xyz2, idx1, gd1, B, N, M, g1, g2, NULL, NULL);
    chamfer_bwd_dir(dt, xyz2, xyz1, idx2, gd2, B, M, N, g2, g1, NULL, NULL);
    return 0;
  }
  double* a1 = (double*)calloc((size_t)(B * N * 3 + 1), sizeof(double));
  double* a2 = (double*)calloc((size_t)(B * M * 3 + 1), sizeof(double));
  if (!a1 || !a2) {
    free(a1);
    free(a2);
    return -3;
  }
  chamfer_bwd_dir(dt, xyz1, xyz2, idx1, gd1, B, N, M, g1, g2, a1, a2);
  chamfer_bwd_dir(dt, xyz2, xyz1, idx2, gd2, B, M, N, g2, g1, a2, a1);
  for (int64_t i = 0; i < B * N * 3; ++i) st(dt, g1, i, rnd(dt, a1[i]));
  for (int64_t i = 0; i < B * M * 3; ++i) st(dt, g2, i, rnd(dt, a2[i]));
  free(a1);
  free(a2);
  return 0;
}

int tpo_ref_chamfer_bwd(int dtype, const void* xyz1, const void* xyz2, const int32_t* idx1,
                        const int32_t* idx2, const void* gd1, const void* gd2, int64_t B,
                        int64_t N, int64_t M, void* gxyz1, void* gxyz2, int accum_f64) {
  if (B < 0 || N < 0 || M < 0) return -1;
  switch (dtype) {
    case TPO_REF_F32: return chamfer_bwd_dt(TPO_REF_F32, xyz1, xyz2, idx1, idx2, gd1, gd2, B, N, M, gxyz1, gxyz2, accum_f64);
    case TPO_REF_F64: return chamfer_bwd_dt(TPO_REF_F64, xyz1, xyz2, idx1, idx2, gd1, gd2, B, N, M, gxyz1, gxyz2, accum_f64);
    case TPO_REF_F16: return chamfer_bwd_dt(TPO_REF_F16, xyz1, xyz2, idx1, idx2, gd1, gd2, B, N, M, gxyz1, gxyz2, accum_f64);
    default: return -2;
  }
}

/* ------------------------------------------------------------------ */
/* KNN                                                                 */
/* ------------------------------------------------------------------ */

/* dispatch.cuh:106-147: V3 for D<=8 && K<=4, V2 for D<=8 && K<=32,
   V1 for D<=32, else V0; explicit invalid versions fall back (knn.cu:332-338). */
static int knn_check_version(int v, int64_t D, int64_t K) {
  if (v == 0) return 1;
  if (v == 1) return D >= 1 && D <= 32;
  if (v == 2) return D >= 1 && D <= 8 && K >= 1 && K <= 32;
  if (v == 3) return D >= 1 && D <= 8 && K >= 1 && K <= 4;
  return 0;
}
int tpo_ref_knn_choose_version(int64_t D, int64_t K, int version) {
  if (version >= 0 && knn_check_version(version, D, K)) return version;
  for (int v = 3; v >= 1; --v)
    if (knn_check_version(v, D, K)) return v;
  return 0;
}

/* Distance of knn.cu:45-57 / 97-107 / 148-158 / 206-216:
   dist = 0; for d: diff = q[d] - r[d]; dist += diff*diff  (norm 2)
                                         dist += |diff|       (norm 1).
   f32/f64 norm 2 under contraction: acc = d0*d0, then acc = fma(dd,dd,acc)
   (fma(d0,d0,0) equals d0*d0, so the first term is the same either way). */
INLINE double knn_dist(int dt, const void* p1, int64_t q0, const void* p2, int64_t r0,
                       int64_t D, int norm) {
  double acc = 0.0;
  for (int64_t d = 0; d < D; ++d) {
    const double diff = op_sub(dt, ld(dt, p1, q0 + d), ld(dt, p2, r0 + d));
    if (norm == 2) {
      if (dt == TPO_REF_F16) acc = op_add(dt, acc, op_mul(dt, diff, diff));
      else acc = (d == 0) ? op_mul(dt, diff, diff) : op_fma(dt, diff, diff, acc);
    } else {
      acc = op_add(dt, acc, diff > 0 ? diff : -diff);
    }
  }
  return acc;
}

/* MinK::add (mink.cuh:89-112): fill slots in order; once full, find the first
   slot holding the maximum (strict-greater scan from slot 0) and replace it
   when the new distance is strictly smaller. */
INLINE void mink_add(double* sd, int64_t* si, int64_t K, int64_t* size, double d, int64_t i) {
  if (*size < K) {
    sd[*size] = d;
    si[*size] = i;
    ++*size;
    return;
  }
  int64_t mi = 0;
  double md = sd[0];
  for (int64_t s = 1; s < K; ++s)
    if (sd[s] > md) {
      md = sd[s];
      mi = s;
    }
  if (d < md) {
    sd[mi] = d;
    si[mi] = i;
  }
}

/* RegisterMinK<.., 2>::add (mink.cuh:221-248): keeps the pair ordered. */
INLINE void mink2_add(double* sd, int64_t* si, int64_t* size, double d, int64_t i) {
  if (*size == 0) {
    sd[0] = d;
    si[0] = i;
    *size = 1;
  } else if (*size == 1) {
    if (d < sd[0]) {
      sd[1] = sd[0];
      si[1] = si[0];
      sd[0] = d;
      si[0] = i;
    } else {
      sd[1] = d;
      si[1] = i;
    }
    *size = 2;
  } else {
    if (d < sd[0]) {
      sd[1] = sd[0];
      si[1] = si[0];
      sd[0] = d;
      si[0] = i;
    } else if (d < sd[1]) {
      sd[1] = d;
      si[1] = i;
    }
  }
}

static int knn_fwd_dt(int dt, const void* p1, const void* p2, const int64_t* len1,
                      const int64_t* len2, int64_t N, int64_t P1, int64_t P2, int64_t D,
                      int64_t K, int norm, int version, int64_t* idxs, void* dists) {
  const int v = tpo_ref_knn_choose_version(D, K, version);
  for (int64_t i = 0; i < N * P1 * K; ++i) {
    idxs[i] = 0;
    st(dt, dists, i, 0.0);
  }
  int err = 0;
  /* every query row is independent: threads change nothing but speed */
#ifdef _OPENMP
#pragma omp parallel
#endif
  {
    double* sd = (double*)malloc((size_t)(K > 0 ? K : 1) * sizeof(double));
    int64_t* si = (int64_t*)malloc((size_t)(K > 0 ? K : 1) * sizeof(int64_t));
    if (!sd || !si) err = 1;
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 16)
#endif
    for (int64_t t = 0; t < N * P1; ++t) {
      if (!sd || !si) continue;
      const int64_t n = t / P1, q = t % P1;
      int64_t l1 = len1[n], l2 = len2[n];
      if (l1 > P1) l1 = P1; /* the reference reads past the cloud here */
      if (l2 > P2) l2 = P2;
      if (q >= l1) continue;
      int64_t size = 0;
      for (int64_t s = 0; s < K; ++s) {
        sd[s] = INFINITY; /* NumericLimits::inf(), mink.cuh:83-86 */
        si[s] = -1;
      }
      for (int64_t r = 0; r < l2; ++r) {
        const double d = knn_dist(dt, p1, (n * P1 + q) * D, p2, (n * P2 + r) * D, D, norm);
        if (v == 3 && K == 2) mink2_add(sd, si, &size, d, r);
        else mink_add(sd, si, K, &size, d, r);
      }
      const int64_t o = (n * P1 + q) * K;
      /* V0/V1 keep MinK in the outputs, so all K slots carry the (inf, -1)
         initialisation (knn.cu:43,95); V2/V3 copy only size() slots
         (knn.cu:163-166, 220-225). */
      const int64_t nw = (v <= 1) ? K : size;
      for (int64_t s = 0; s < nw; ++s) {
        idxs[o + s] = si[s];
        st(dt, dists, o + s, sd[s]);
      }
    }
    free(sd);
    free(si);
  }
  return err ? -3 : 0;
}

int tpo_ref_knn_fwd(int dtype, const void* p1, const void* p2, const int64_t* len1,
                    const int64_t* len2, int64_t N, int64_t P1, int64_t P2, int64_t D,
                    int64_t K, int norm, int version, int64_t* idxs, void* dists) {
  if (N < 0 || P1 < 0 || P2 < 0 || D < 1 || K < 1 || (norm != 1 && norm != 2)) return -1;
  switch (dtype) {
    case TPO_REF_F32: return knn_fwd_dt(TPO_REF_F32, p1, p2, len1, len2, N, P1, P2, D, K, norm, version, idxs, dists);
    case TPO_REF_F64: return knn_fwd_dt(TPO_REF_F64, p1, p2, len1, len2, N, P1, P2, D, K, norm, version, idxs, dists);
    case TPO_REF_F16: return knn_fwd_dt(TPO_REF_F16, p1, p2, len1, len2, N, P1, P2, D, K, norm, version, idxs, dists);
    default: return -2;
  }
}

/* knn.cu:400-466: rows q < len1, slots with idx != -1;
   L2: diff = (2*g)*(p1 - p2); L1: diff = g*sign, sign 0 when equal (:445-448);
   grad_p1 += diff, grad_p2[idx] += -diff. */
static int knn_bwd_dt(int dt, const void* p1, const void* p2, const int64_t* len1,
                      const int64_t* len2, const int64_t* idxs, int norm, const void* gdist,
                      int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K, void* gp1,
                      void* gp2, int accum_f64) {
  (void)len2;
  double* a1 = NULL;
  double* a2 = NULL;
  if (accum_f64) {
    a1 = (double*)calloc((size_t)(N * P1 * D + 1), sizeof(double));
    a2 = (double*)calloc((size_t)(N * P2 * D + 1), sizeof(double));
    if (!a1 || !a2) {
      free(a1);
      free(a2);
      return -3;
    }
  }
  for (int64_t i = 0; i < N * P1 * D; ++i) st(dt, gp1, i, 0.0);
  for (int64_t i = 0; i < N * P2 * D; ++i) st(dt, gp2, i, 0.0);
  for (int64_t n = 0; n < N; ++n) {
    int64_t l1 = len1[n];
    if (l1 > P1) l1 = P1;
    for (int64_t q = 0; q < l1; ++q) {
      for (int64_t k = 0; k < K; ++k) {
        const int64_t r = idxs[(n * P1 + q) * K + k];
        if (r == -1) continue;
        if (r < 0 || r >= P2) continue; /* the reference would read out of bounds */
        const double g = ld(dt, gdist, (n * P1 + q) * K + k);
        for (int64_t d = 0; d < D; ++d) {
          const int64_t i1 = (n * P1 + q) * D + d, i2 = (n * P2 + r) * D + d;
          const double v1 = ld(dt, p1, i1), v2 = ld(dt, p2, i2);
          double diff;
          if (norm == 1) {
            const double sign = (v1 > v2) ? 1.0 : (v1 == v2 ? 0.0 : -1.0);
            diff = op_mul(dt, g, sign);
          } else {
            diff = op_mul(dt, op_mul(dt, 2.0, g), op_sub(dt, v1, v2));
          }
          if (accum_f64) {
            a1[i1] += diff;
            a2[i2] -= diff;
          } else {
            st(dt, gp1, i1, op_add(dt, ld(dt, gp1, i1), diff));
            st(dt, gp2, i2, op_add(dt, ld(dt, gp2, i2), -diff));
          }
        }
      }
    }
  }
  if (accum_f64) {
    for (int64_t i = 0; i < N * P1 * D; ++i) st(dt, gp1, i, rnd(dt, a1[i]));
    for (int64_t i = 0; i < N * P2 * D; ++i) st(dt, gp2, i, rnd(dt, a2[i]));
    free(a1);
    free(a2);
  }
  return 0;
}

int tpo_ref_knn_bwd(int dtype, const void* p1, const void* p2, const int64_t* len1,
                    const int64_t* len2, const int64_t* idxs, int norm, const void* grad_dists,
                    int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K, void* gp1,
                    void* gp2, int accum_f64) {
  if (N < 0 || P1 < 0 || P2 < 0 || D < 1 || K < 0 || (norm != 1 && norm != 2)) return -1;
  switch (dtype) {
    case TPO_REF_F32: return knn_bwd_dt(TPO_REF_F32, p1, p2, len1, len2, idxs, norm, grad_dists, N, P1, P2, D, K, gp1, gp2, accum_f64);
    case TPO_REF_F64: return knn_bwd_dt(TPO_REF_F64, p1, p2, len1, len2, idxs, norm, grad_dists, N, P1, P2, D, K, gp1, gp2, accum_f64);
    case TPO_REF_F16: return knn_bwd_dt(TPO_REF_F16, p1, p2, len1, len2, idxs, norm, grad_dists, N, P1, P2, D, K, gp1, gp2, accum_f64);
    default: return -2;
  }
}

/* ------------------------------------------------------------------ */
/* FPS                                                                 */
/* ------------------------------------------------------------------ */

/* fps.cu:56-60: min(512, 2^floor(log2 n)) */
int tpo_ref_fps_block_size(int64_t n) {
  if (n <= 0) return 1;
  int bs = 1;
  while ((int64_t)bs * 2 <= n && bs < 512) bs *= 2;
  return bs;
}

int64_t tpo_ref_fps_rank(int64_t k, int64_t n) {
  const int64_t bs = tpo_ref_fps_block_size(n);
  int bits = 0;
  while ((1 << bits) < bs) ++bits;
  const int64_t t = k % bs;
  int64_t rev = 0;
  for (int i = 0; i < bits; ++i)
    if (t & (1 << i)) rev |= (int64_t)1 << (bits - 1 - i);
  const int64_t per = (n + bs - 1) / bs;
  return rev * per + k / bs;
}

/* fps.cu:111-214, one cloud at a time, with the block's threads simulated in
   order: each thread tid sweeps k = tid, tid+BS, ... skipping points whose
   magnitude is not > 1e-3 (:142-143), updates temp[k] = min(d, temp[k])
   (:145-147) and keeps the first strictly greater value (:148-149); then the
   shared-memory tree (:151-209) with __update (:100-108) picks the winner.
   temp starts at 1e10 (1e4 for fp16) (fps.cu:291-292). */
static int fps_dt(int dt, const void* pts, int64_t B, int64_t N, int64_t m, int64_t* idx) {
  const int bs = tpo_ref_fps_block_size(N);
  /* scalar_t(1e-3): the double literal converts to float, then to the dtype */
  const double thr = (dt == TPO_REF_F64) ? 1e-3 : (dt == TPO_REF_F16 ? rh(1e-3f) : (double)1e-3f);
  const double init = (dt == TPO_REF_F16) ? 1e4 : 1e10;
  int err = 0;
  /* clouds are independent: threads change nothing but speed */
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1)
#endif
  for (int64_t b = 0; b < B; ++b) {
    double* temp = (double*)malloc((size_t)(N > 0 ? N : 1) * sizeof(double));
    double* mag = (double*)malloc((size_t)(N > 0 ? N : 1) * sizeof(double));
    double* dv = (double*)malloc((size_t)bs * sizeof(double));
    int64_t* di = (int64_t*)malloc((size_t)bs * sizeof(int64_t));
    if (!temp || !mag || !dv || !di) {
      err = 1;
      free(temp);
      free(mag);
      free(dv);
      free(di);
      continue;
    }
    const int64_t base = b * N * 3;
    for (int64_t k = 0; k < N; ++k) {
      temp[k] = init;
      mag[k] = sq3(dt, ld(dt, pts, base + 3 * k), ld(dt, pts, base + 3 * k + 1),
                   ld(dt, pts, base + 3 * k + 2));
    }
    int64_t old = 0;
    if (m > 0) idx[b * m] = 0;
    for (int64_t j = 1; j < m; ++j) {
      const double x1 = ld(dt, pts, base + 3 * old), y1 = ld(dt, pts, base + 3 * old + 1),
                   z1 = ld(dt, pts, base + 3 * old + 2);
      for (int tid = 0; tid < bs; ++tid) {
        int64_t besti = 0;
        double best = -1.0;
        for (int64_t k = tid; k < N; k += bs) {
          if (!(mag[k] > thr)) continue;
          const double x2 = ld(dt, pts, base + 3 * k), y2 = ld(dt, pts, base + 3 * k + 1),
                       z2 = ld(dt, pts, base + 3 * k + 2);
          const double d = sq3(dt, op_sub(dt, x2, x1), op_sub(dt, y2, y1), op_sub(dt, z2, z1));
          const double d2 = d < temp[k] ? d : temp[k];
          temp[k] = d2;
          if (d2 > best) {
            besti = k;
            best = d2;
          }
        }
        dv[tid] = best;
        di[tid] = besti;
      }
      for (int s = bs / 2; s >= 1; s /= 2) {
        for (int t = 0; t < s; ++t) {
          const double v1 = dv[t], v2 = dv[t + s];
          const int64_t i1 = di[t], i2 = di[t + s];
          dv[t] = v1 > v2 ? v1 : v2;
          di[t] = v2 > v1 ? i2 : i1;
        }
      }
      old = di[0];
      idx[b * m + j] = old;
    }
    free(temp);
    free(mag);
    free(dv);
    free(di);
  }
  return err ? -3 : 0;
}

int tpo_ref_fps(int dtype, const void* pts, int64_t B, int64_t N, int64_t m, int64_t* idx) {
  if (B < 0 || N < 1 || m < 1 || m > N) return -1;
  switch (dtype) {
    case TPO_REF_F32: return fps_dt(TPO_REF_F32, pts, B, N, m, idx);
    case TPO_REF_F64: return fps_dt(TPO_REF_F64, pts, B, N, m, idx);
    case TPO_REF_F16: return fps_dt(TPO_REF_F16, pts, B, N, m, idx);
    default: return -2;
  }
}

/* ------------------------------------------------------------------ */
/* gather_points                                                       */
/* ------------------------------------------------------------------ */

/* fps.cu:63-76: out[b,c,j] = pts[b,c,idx[b,j]] (no bounds check there; the
   oracle rejects out-of-range indices instead). */
int tpo_ref_gather_fwd(int dtype, const void* pts, const int64_t* idx, int64_t B, int64_t C,
                       int64_t N, int64_t M, void* out) {
  const int64_t esz = (dtype == TPO_REF_F64) ? 8 : (dtype == TPO_REF_F32 ? 4 : 2);
  for (int64_t b = 0; b < B; ++b)
    for (int64_t j = 0; j < M; ++j)
      if (idx[b * M + j] < 0 || idx[b * M + j] >= N) return -4;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t c = 0; c < C; ++c)
      for (int64_t j = 0; j < M; ++j)
        memcpy((char*)out + ((b * C + c) * M + j) * esz,
               (const char*)pts + ((b * C + c) * N + idx[b * M + j]) * esz, (size_t)esz);
  return 0;
}

/* fps.cu:79-98 + :376: zeros(B,C,N), then grad_pts[b,c,idx[b,j]] += grad_out[b,c,j]. */
static int gather_bwd_dt(int dt, const void* go, const int64_t* idx, int64_t B, int64_t C,
                         int64_t N, int64_t M, void* gp, int accum_f64) {
  double* acc = NULL;
  if (accum_f64) {
    acc = (double*)calloc((size_t)(B * C * N + 1), sizeof(double));
    if (!acc) return -3;
  }
  for (int64_t i = 0; i < B * C * N; ++i) st(dt, gp, i, 0.0);
  for (int64_t b = 0; b < B; ++b)
    for (int64_t c = 0; c < C; ++c)
      for (int64_t j = 0; j < M; ++j) {
        const int64_t a = idx[b * M + j];
        if (a < 0 || a >= N) continue;
        const int64_t o = (b * C + c) * N + a;
        const double g = ld(dt, go, (b * C + c) * M + j);
        if (accum_f64) acc[o] += g;
        else st(dt, gp, o, op_add(dt, ld(dt, gp, o), g));
      }
  if (accum_f64) {
    for (int64_t i = 0; i < B * C * N; ++i) st(dt, gp, i, rnd(dt, acc[i]));
    free(acc);
  }
  return 0;
}

int tpo_ref_gather_bwd(int dtype, const void* grad_out, const int64_t* idx, int64_t B,
                       int64_t C, int64_t N, int64_t M, void* grad_pts, int accum_f64) {
  switch (dtype) {
    case TPO_REF_F32: return gather_bwd_dt(TPO_REF_F32, grad_out, idx, B, C, N, M, grad_pts, accum_f64);
    case TPO_REF_F64: return gather_bwd_dt(TPO_REF_F64, grad_out, idx, B, C, N, M, grad_pts, accum_f64);
    case TPO_REF_F16: return gather_bwd_dt(TPO_REF_F16, grad_out, idx, B, C, N, M, grad_pts, accum_f64);
    default: return -2;
  }
}

/* ------------------------------------------------------------------ */
/* Earth mover's distance                                              */
/* ------------------------------------------------------------------ */

/* emd.cu computes in at::opmath_type (float for float32 and float16, double
   for float64); every opmath operation below rounds to it.  The remain,
   ratio and match arrays are scalar_t, so float16 stores round to binary16
   (om_st).  Contractions follow the same rule as the distances above:
   a*a + b*b + c*c -> fma(c,c, fma(a,a, b*b)) and s += e*w -> fma(e,w,s). */
INLINE int om64(int dt) { return dt == TPO_REF_F64; }
INLINE double om_add(int dt, double a, double b) { return om64(dt) ? a + b : (double)((float)a + (float)b); }
INLINE double om_sub(int dt, double a, double b) { return om64(dt) ? a - b : (double)((float)a - (float)b); }
INLINE double om_mul(int dt, double a, double b) { return om64(dt) ? a * b : (double)((float)a * (float)b); }
INLINE double om_div(int dt, double a, double b) { return om64(dt) ? a / b : (double)((float)a / (float)b); }
INLINE double om_fma(int dt, double a, double b, double c) {
  return om64(dt) ? fma(a, b, c) : (double)fmaf((float)a, (float)b, (float)c);
}
INLINE double om_exp(int dt, double x) { return om64(dt) ? exp(x) : (double)expf((float)x); }
INLINE double om_st(int dt, double v) { return dt == TPO_REF_F16 ? rh((float)v) : v; }
/* fminf/fmaxf are float functions: emd.cu:134,136,178 pass them opmath
   values, so a float64 argument is narrowed to float there. */
INLINE double om_fminf(double a, float b) { return (double)fminf((float)a, b); }
INLINE double om_fmaxf(float a, double b) { return (double)fmaxf(a, (float)b); }

/* (x2-x1)^2 + (y2-y1)^2 + (z2-z1)^2, emd.cu:72,120,164,212 */
INLINE double emd_sq(int dt, const double* p1, const double* p2) {
  const double a = om_sub(dt, p2[0], p1[0]), b = om_sub(dt, p2[1], p1[1]),
               c = om_sub(dt, p2[2], p1[2]);
  return om_fma(dt, c, c, om_fma(dt, a, a, om_mul(dt, b, b)));
}
/* exp(level * d), with the float16 clamp of emd.cu:77-80 */
INLINE double emd_e(int dt, double level, const double* p1, const double* p2) {
  double d = om_mul(dt, level, emd_sq(dt, p1, p2));
  if (dt == TPO_REF_F16) d = d < -20.0 ? -20.0 : (d > 20.0 ? 20.0 : d);
  return om_exp(dt, d);
}

/* One cloud of approxmatch (emd.cu:18-183) followed by matchcost
   (emd.cu:187-230).  The reference's 1024-point staging tiles do not change
   any summation order, so the loops run straight over the points. */
static void emd_fwd_one(int dt, const void* xyz1, const void* xyz2, int64_t b, int64_t n,
                        int64_t m, void* cost, void* match_out) {
  double* X1 = (double*)malloc(sizeof(double) * (size_t)(3 * n + 3 * m + 3 * (n + m) + n * m));
  double* X2 = X1 + 3 * n;
  double* remL = X2 + 3 * m;
  double* remR = remL + n;
  double* ratL = remR + m;
  double* ratR = ratL + n;
  double* match = ratR + m;
  for (int64_t i = 0; i < 3 * n; ++i) X1[i] = ld(dt, xyz1, b * n * 3 + i);
  for (int64_t i = 0; i < 3 * m; ++i) X2[i] = ld(dt, xyz2, b * m * 3 + i);
  /* emd.cu:55,89: static_cast<opmath_t>(1e-9f), or 1e-4f for float16 */
  const double eps = dt == TPO_REF_F16 ? (double)1e-4f : (double)1e-9f;
  /* emd.cu:21-28: float(n)/m, stored as scalar_t */
  double multiL = 1.0, multiR = 1.0;
  if (n >= m) multiR = om_st(dt, (double)((float)n / (float)m));
  else multiL = om_st(dt, (double)((float)m / (float)n));
  for (int64_t i = 0; i < n * m; ++i) match[i] = 0.0;
  for (int64_t k = 0; k < n; ++k) remL[k] = multiL;
  for (int64_t l = 0; l < m; ++l) remR[l] = multiR;
  for (int j = 7; j >= -2; --j) {
    const double level = j == -2 ? 0.0 : -pow(4.0, j);  /* emd.cu:40-43, exact in float */
    for (int64_t k = 0; k < n; ++k) {                   /* emd.cu:47-96 */
      double suml = eps;
      for (int64_t l = 0; l < m; ++l)
        suml = om_fma(dt, emd_e(dt, level, X1 + 3 * k, X2 + 3 * l), remR[l], suml);
      ratL[k] = om_st(dt, om_div(dt, remL[k], om_add(dt, suml, eps)));
    }
    for (int64_t l = 0; l < m; ++l) {                   /* emd.cu:98-138 */
      double sumr = 0.0;
      for (int64_t k = 0; k < n; ++k)
        sumr = om_fma(dt, emd_e(dt, level, X1 + 3 * k, X2 + 3 * l), ratL[k], sumr);
      sumr = om_mul(dt, sumr, remR[l]);
      const double cons = om_fminf(om_div(dt, remR[l], om_add(dt, sumr, eps)), 1.0f);
      ratR[l] = om_st(dt, om_mul(dt, cons, remR[l]));
      remR[l] = om_st(dt, om_fmaxf(0.0f, om_sub(dt, remR[l], sumr)));
    }
    for (int64_t k = 0; k < n; ++k) {                   /* emd.cu:140-179 */
      const double rl = ratL[k];
      double suml = 0.0;
      for (int64_t l = 0; l < m; ++l) {
        const double w =
            om_mul(dt, om_mul(dt, emd_e(dt, level, X1 + 3 * k, X2 + 3 * l), rl), ratR[l]);
        match[l * n + k] = om_st(dt, om_add(dt, match[l * n + k], om_st(dt, w)));
        suml = om_add(dt, suml, w);
      }
      remL[k] = om_st(dt, om_fmaxf(0.0f, om_sub(dt, remL[k], suml)));
    }
  }
  /* matchcost: thread t of 512 sums its columns k = t, t+512, ... over l in
     order, then the block's tree (emd.cu:193-227) */
  double part[512];
  for (int t = 0; t < 512; ++t) {
    double s = 0.0;
    for (int64_t k = t; k < n; k += 512)
      for (int64_t l = 0; l < m; ++l)
        s = om_fma(dt, emd_sq(dt, X1 + 3 * k, X2 + 3 * l), match[l * n + k], s);
    part[t] = s;
  }
  for (int st2 = 1; st2 < 512; st2 <<= 1)
    for (int t = 0; t + st2 < 512; t += 2 * st2) part[t] = om_add(dt, part[t], part[t + st2]);
  st(dt, cost, b, om_st(dt, part[0]));
  for (int64_t i = 0; i < n * m; ++i) st(dt, match_out, b * n * m + i, match[i]);
  free(X1);
}

int tpo_ref_emd_fwd(int dtype, const void* xyz1, const void* xyz2, int64_t B, int64_t n,
                    int64_t m, void* cost, void* match) {
  if (dtype != TPO_REF_F32 && dtype != TPO_REF_F64 && dtype != TPO_REF_F16) return -2;
  if (B < 0 || n < 0 || m < 0) return -1;
  if (n == 0 || m == 0) { /* emd.cu:313-318 */
    for (int64_t b = 0; b < B; ++b) st(dtype, cost, b, 0.0);
    return 0;
  }
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t b = 0; b < B; ++b) emd_fwd_one(dtype, xyz1, xyz2, b, n, m, cost, match);
  return 0;
}

/* matchcostgrad1 (emd.cu:234-257) and matchcostgrad2 (emd.cu:261-303) */
int tpo_ref_emd_bwd(int dtype, const void* grad_cost, const void* xyz1, const void* xyz2,
                    const void* match, int64_t B, int64_t n, int64_t m, void* grad1,
                    void* grad2) {
  const int dt = dtype;
  if (dt != TPO_REF_F32 && dt != TPO_REF_F64 && dt != TPO_REF_F16) return -2;
  if (B < 0 || n < 0 || m < 0) return -1;
  if (n == 0 || m == 0) {
    for (int64_t i = 0; i < B * n * 3; ++i) st(dt, grad1, i, 0.0);
    for (int64_t i = 0; i < B * m * 3; ++i) st(dt, grad2, i, 0.0);
    return 0;
  }
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t b = 0; b < B; ++b) {
    const double g = ld(dt, grad_cost, b);
    for (int64_t l = 0; l < n; ++l) {
      double p1[3], acc[3] = {0.0, 0.0, 0.0};
      for (int c = 0; c < 3; ++c) p1[c] = ld(dt, xyz1, (b * n + l) * 3 + c);
      for (int64_t k = 0; k < m; ++k) {
        const double d = om_mul(dt, ld(dt, match, b * n * m + k * n + l), 2.0);
        for (int c = 0; c < 3; ++c)
          acc[c] = om_fma(dt, om_sub(dt, p1[c], ld(dt, xyz2, (b * m + k) * 3 + c)), d, acc[c]);
      }
      for (int c = 0; c < 3; ++c) st(dt, grad1, (b * n + l) * 3 + c, om_st(dt, om_mul(dt, acc[c], g)));
    }
    for (int64_t k = 0; k < m; ++k) {
      double p2[3], part[256][3];
      for (int c = 0; c < 3; ++c) p2[c] = ld(dt, xyz2, (b * m + k) * 3 + c);
      for (int t = 0; t < 256; ++t) {
        double s[3] = {0.0, 0.0, 0.0};
        for (int64_t jj = t; jj < n; jj += 256) {
          const double d = om_mul(dt, ld(dt, match, b * n * m + k * n + jj), 2.0);
          for (int c = 0; c < 3; ++c)
            s[c] = om_fma(dt, om_sub(dt, p2[c], ld(dt, xyz1, (b * n + jj) * 3 + c)), d, s[c]);
        }
        for (int c = 0; c < 3; ++c) part[t][c] = s[c];
      }
      for (int st2 = 1; st2 < 256; st2 <<= 1)
        for (int t = 0; t + st2 < 256; t += 2 * st2)
          for (int c = 0; c < 3; ++c) part[t][c] = om_add(dt, part[t][c], part[t + st2][c]);
      for (int c = 0; c < 3; ++c) st(dt, grad2, (b * m + k) * 3 + c, om_st(dt, om_mul(dt, part[0][c], g)));
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* Reference CPU kernels (knn.cpp, fps.cpp)                            */
/* ------------------------------------------------------------------ */

/* These restate the reference's CPU dispatch-key kernels, whose arithmetic
   differs from the CUDA kernels': the reference builds them with g++ -O3 for
   plain x86-64 (setup.py:78-81), which has no FMA instruction, so every
   distance sum rounds after each + and *; float16 uses c10::Half's operators
   (one rounding per operation).  They are the checker of the product's CPU
   kernels and the timed CPU baseline.  nthreads > 1 splits independent rows
   or clouds over OpenMP threads; the result does not depend on it. */

/* std::priority_queue<std::tuple<scalar_t,int>> (knn.cpp:60) is a max-heap
   under std::tuple's operator<: a < b iff a.d < b.d, or neither distance is
   less than the other and a.i < b.i. */
typedef struct {
  double d;
  int i;
} knn_item;
static inline int item_lt(knn_item a, knn_item b) {
  return a.d < b.d || (!(b.d < a.d) && a.i < b.i);
}
static void heap_push(knn_item* h, int* n, knn_item v) {
  int c = (*n)++;
  h[c] = v;
  while (c > 0) {
    int p = (c - 1) / 2;
    if (!item_lt(h[p], h[c])) break;
    knn_item t = h[p];
    h[p] = h[c];
    h[c] = t;
    c = p;
  }
}
static void heap_pop(knn_item* h, int* n) {
  h[0] = h[--*n];
  int c = 0;
  for (;;) {
    int l = 2 * c + 1, r = l + 1, g = c;
    if (l < *n && item_lt(h[g], h[l])) g = l;
    if (r < *n && item_lt(h[g], h[r])) g = r;
    if (g == c) break;
    knn_item t = h[g];
    h[g] = h[c];
    h[c] = t;
    c = g;
  }
}

static int64_t clamp_len(int64_t v, int64_t hi) { return v < 0 ? 0 : (v > hi ? hi : v); }

/* knn.cpp:30-99: idxs preset to -1 and dists to 0; for each query q <
   lengths1 a heap of the K smallest (dist, idx) over p2[0:lengths2]: a
   reference enters while the heap holds fewer than K, or when its distance
   is strictly below the top's (then the top is popped); the heap is emptied
   into the row in ascending order (:82-93).  dist = 0; dist += diff*diff
   (or |diff|) per coordinate, rounded after each operation.  Lengths are
   clamped to the cloud sizes (the reference reads past the cloud). */
static int cpu_knn_fwd_dt(int dt, const void* p1, const void* p2, const int64_t* len1,
                          const int64_t* len2, int64_t N, int64_t P1, int64_t P2, int64_t D,
                          int64_t K, int norm, int64_t* idxs, void* dists, int nthreads) {
  for (int64_t i = 0; i < N * P1 * K; ++i) {
    idxs[i] = -1;
    st(dt, dists, i, 0.0);
  }
  const int64_t total = N * P1;
  int err = 0;
#ifdef _OPENMP
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
#else
  (void)nthreads;
#endif
  {
    knn_item* h = (knn_item*)malloc((size_t)(K + 1) * sizeof(knn_item));
    if (!h) err = 1;
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 16)
#endif
    for (int64_t t = 0; t < total; ++t) {
      if (!h) continue;
      const int64_t n = t / P1, q = t % P1;
      if (q >= clamp_len(len1[n], P1)) continue;
      const int64_t l2 = clamp_len(len2[n], P2);
      int hn = 0;
      for (int64_t r = 0; r < l2; ++r) {
        double dist = 0.0;
        for (int64_t d = 0; d < D; ++d) {
          const double diff =
              op_sub(dt, ld(dt, p1, (n * P1 + q) * D + d), ld(dt, p2, (n * P2 + r) * D + d));
          dist = op_add(dt, dist, norm == 1 ? fabs(diff) : op_mul(dt, diff, diff));
        }
        if (hn < K || dist < h[0].d) {
          knn_item it = {dist, (int)r};
          heap_push(h, &hn, it);
          if (hn > K) heap_pop(h, &hn);
        }
      }
      const int64_t o = (n * P1 + q) * K;
      for (int64_t k = hn - 1; k >= 0; --k) { /* the top is the largest: fill from the back */
        st(dt, dists, o + k, h[0].d);
        idxs[o + k] = h[0].i;
        heap_pop(h, &hn);
      }
    }
    free(h);
  }
  return err ? -3 : 0;
}

int tpo_cpu_knn_fwd(int dtype, const void* p1, const void* p2, const int64_t* len1,
                    const int64_t* len2, int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K,
                    int norm, int64_t* idxs, void* dists, int nthreads) {
  if (N < 0 || P1 < 0 || P2 < 0 || K < 1 || D < 1 || (norm != 1 && norm != 2)) return -1;
  switch (dtype) {
    case TPO_REF_F32: return cpu_knn_fwd_dt(TPO_REF_F32, p1, p2, len1, len2, N, P1, P2, D, K, norm, idxs, dists, nthreads);
    case TPO_REF_F64: return cpu_knn_fwd_dt(TPO_REF_F64, p1, p2, len1, len2, N, P1, P2, D, K, norm, idxs, dists, nthreads);
    case TPO_REF_F16: return cpu_knn_fwd_dt(TPO_REF_F16, p1, p2, len1, len2, N, P1, P2, D, K, norm, idxs, dists, nthreads);
    default: return -2;
  }
}

/* knn.cpp:104-164: gradients start at zero; for each cloud, rows q <
   lengths1, slots k < min(lengths2, K) whose index is not -1, coordinates
   d in order:
     norm 1: sign = p1 > p2 ? 1 : -1 (-1 on equality, :150), diff = g*sign;
     norm 2: diff = 2.0*g*(p1 - p2), the product taken in double (2.0 is a
             double literal) and rounded once to the dtype when stored;
   grad_p1[q] += diff, grad_p2[idx] -= diff, in this loop order (sequential:
   the sums are order-dependent).  Indices outside [0, P2) other than -1
   are skipped (the reference would access out of bounds).  Threads split
   the clouds. */
static int cpu_knn_bwd_dt(int dt, const void* p1, const void* p2, const int64_t* len1,
                          const int64_t* len2, const int64_t* idxs, int norm, const void* gdist,
                          int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K, void* gp1,
                          void* gp2, int nthreads) {
  for (int64_t i = 0; i < N * P1 * D; ++i) st(dt, gp1, i, 0.0);
  for (int64_t i = 0; i < N * P2 * D; ++i) st(dt, gp2, i, 0.0);
#ifdef _OPENMP
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(dynamic, 1)
#else
  (void)nthreads;
#endif
  for (int64_t n = 0; n < N; ++n) {
    const int64_t l1 = clamp_len(len1[n], P1);
    int64_t l2 = len2[n] < K ? len2[n] : K;
    for (int64_t q = 0; q < l1; ++q)
      for (int64_t k = 0; k < l2; ++k) {
        const int64_t r = idxs[(n * P1 + q) * K + k];
        if (r == -1 || r < 0 || r >= P2) continue;
        const double g = ld(dt, gdist, (n * P1 + q) * K + k);
        for (int64_t d = 0; d < D; ++d) {
          const int64_t i1 = (n * P1 + q) * D + d, i2 = (n * P2 + r) * D + d;
          const double v1 = ld(dt, p1, i1), v2 = ld(dt, p2, i2);
          double diff;
          if (norm == 1) diff = op_mul(dt, g, v1 > v2 ? 1.0 : -1.0);
          else diff = rnd(dt, (2.0 * g) * op_sub(dt, v1, v2));
          st(dt, gp1, i1, op_add(dt, ld(dt, gp1, i1), diff));
          st(dt, gp2, i2, op_sub(dt, ld(dt, gp2, i2), diff));
        }
      }
  }
  return 0;
}

int tpo_cpu_knn_bwd(int dtype, const void* p1, const void* p2, const int64_t* len1,
                    const int64_t* len2, const int64_t* idxs, int norm, const void* grad_dists,
                    int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K, void* gp1, void* gp2,
                    int nthreads) {
  if (N < 0 || P1 < 0 || P2 < 0 || K < 0 || D < 1 || (norm != 1 && norm != 2)) return -1;
  switch (dtype) {
    case TPO_REF_F32: return cpu_knn_bwd_dt(TPO_REF_F32, p1, p2, len1, len2, idxs, norm, grad_dists, N, P1, P2, D, K, gp1, gp2, nthreads);
    case TPO_REF_F64: return cpu_knn_bwd_dt(TPO_REF_F64, p1, p2, len1, len2, idxs, norm, grad_dists, N, P1, P2, D, K, gp1, gp2, nthreads);
    case TPO_REF_F16: return cpu_knn_bwd_dt(TPO_REF_F16, p1, p2, len1, len2, idxs, norm, grad_dists, N, P1, P2, D, K, gp1, gp2, nthreads);
    default: return -2;
  }
}

/* x*x + y*y + z*z of fps.cpp:57,64 without contraction: ((x*x + y*y) + z*z). */
INLINE double cpu_sq3(int dt, double x, double y, double z) {
  return op_add(dt, op_add(dt, op_mul(dt, x, x), op_mul(dt, y, y)), op_mul(dt, z, z));
}

/* fps.cpp:18-88 (the CPU semantics, unlike fps.cu's): min distances start at
   numeric_limits<scalar_t>::max(); index 0 first; each iteration updates the
   unselected points whose |p|^2 is not <= scalar_t(1e-3) with
   min(min_dist, dist) (std::min keeps the old value unless the new one is
   strictly smaller), then picks the first unselected point with the
   strictly greatest min distance (start -1, index 0 when none). */
static int cpu_fps_dt(int dt, const void* pts, int64_t B, int64_t N, int64_t m, int64_t* idx,
                      int nthreads) {
  const double big = dt == TPO_REF_F64 ? 1.7976931348623157e308
                                       : (dt == TPO_REF_F16 ? 65504.0 : 3.4028234663852886e38);
  const double thr = dt == TPO_REF_F64 ? 1e-3 : (dt == TPO_REF_F16 ? rh(1e-3f) : (double)1e-3f);
  int err = 0;
#ifdef _OPENMP
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(dynamic, 1)
#else
  (void)nthreads;
#endif
  for (int64_t b = 0; b < B; ++b) {
    double* md = (double*)malloc((size_t)N * sizeof(double));
    unsigned char* sel = (unsigned char*)calloc((size_t)N, 1);
    if (!md || !sel) {
      err = 1;
      free(md);
      free(sel);
      continue;
    }
    const int64_t base = b * N * 3;
    for (int64_t k = 0; k < N; ++k) md[k] = big;
    int64_t cur = 0;
    idx[b * m] = 0;
    sel[0] = 1;
    for (int64_t i = 1; i < m; ++i) {
      const double cx = ld(dt, pts, base + 3 * cur), cy = ld(dt, pts, base + 3 * cur + 1),
                   cz = ld(dt, pts, base + 3 * cur + 2);
      for (int64_t j = 0; j < N; ++j) {
        if (sel[j]) continue;
        const double x = ld(dt, pts, base + 3 * j), y = ld(dt, pts, base + 3 * j + 1),
                     z = ld(dt, pts, base + 3 * j + 2);
        if (cpu_sq3(dt, x, y, z) <= thr) continue;
        const double dist = cpu_sq3(dt, op_sub(dt, x, cx), op_sub(dt, y, cy), op_sub(dt, z, cz));
        md[j] = dist < md[j] ? dist : md[j];
      }
      double best = -1.0;
      int64_t bi = 0;
      for (int64_t j = 0; j < N; ++j)
        if (!sel[j] && md[j] > best) {
          best = md[j];
          bi = j;
        }
      cur = bi;
      idx[b * m + i] = cur;
      sel[cur] = 1;
    }
    free(md);
    free(sel);
  }
  return err ? -3 : 0;
}

int tpo_cpu_fps(int dtype, const void* pts, int64_t B, int64_t N, int64_t m, int64_t* idx,
                int nthreads) {
  if (B < 0 || N < 1 || m < 1 || m > N) return -1;
  switch (dtype) {
    case TPO_REF_F32: return cpu_fps_dt(TPO_REF_F32, pts, B, N, m, idx, nthreads);
    case TPO_REF_F64: return cpu_fps_dt(TPO_REF_F64, pts, B, N, m, idx, nthreads);
    case TPO_REF_F16: return cpu_fps_dt(TPO_REF_F16, pts, B, N, m, idx, nthreads);
    default: return -2;
  }
}

/* fps.cpp:91-115: out[b,c,j] = pts[b,c,idx[b,j]]; an index outside [0, N)
   gives 0 here (the reference reads out of bounds). */
int tpo_cpu_gather_fwd(int dtype, const void* pts, const int64_t* idx, int64_t B, int64_t C,
                       int64_t N, int64_t M, void* out) {
  if (dtype < TPO_REF_F32 || dtype > TPO_REF_F16) return -2;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t c = 0; c < C; ++c)
      for (int64_t j = 0; j < M; ++j) {
        const int64_t a = idx[b * M + j];
        st(dtype, out, (b * C + c) * M + j, (a < 0 || a >= N) ? 0.0 : ld(dtype, pts, (b * C + c) * N + a));
      }
  return 0;
}

/* fps.cpp:118-141: zeros, then grad_pts[b,c,idx[b,j]] += grad_out[b,c,j] in
   (b, c, j) order, rounded to the dtype at every addition; indices outside
   [0, N) are skipped. */
int tpo_cpu_gather_bwd(int dtype, const void* grad_out, const int64_t* idx, int64_t B, int64_t C,
                       int64_t N, int64_t M, void* grad_pts) {
  if (dtype < TPO_REF_F32 || dtype > TPO_REF_F16) return -2;
  for (int64_t i = 0; i < B * C * N; ++i) st(dtype, grad_pts, i, 0.0);
  for (int64_t b = 0; b < B; ++b)
    for (int64_t c = 0; c < C; ++c)
      for (int64_t j = 0; j < M; ++j) {
        const int64_t a = idx[b * M + j];
        if (a < 0 || a >= N) continue;
        const int64_t o = (b * C + c) * N + a;
        st(dtype, grad_pts, o, op_add(dtype, ld(dtype, grad_pts, o), ld(dtype, grad_out, (b * C + c) * M + j)));
      }
  return 0;
}
