// cpu_ops.cpp -- the CPU dispatch-key kernels of torch_point_ops: knn_forward,
// knn_backward, fps_forward, gather_points_forward/backward and
// quick_fps_forward on host tensors.
//
// They reproduce the reference's CPU kernels bit for bit
//   knn_cpu_forward            knn.cpp:30-99
//   knn_cpu_backward           knn.cpp:104-164
//   fps_cpu_forward            fps.cpp:18-88
//   gather_points_cpu_forward  fps.cpp:91-115
//   gather_points_cpu_backward fps.cpp:118-141
//   quick_fps_cpu_forward      fps.cpp:144-155
// including their arithmetic: every + and * rounds (no fused multiply-add;
// this file is compiled with -ffp-contract=off, and the reference's plain
// x86-64 build has no FMA), c10::Half operators round after each operation,
// and the CPU semantics differ from the GPU kernels' on purpose (KNN padding
// idx -1; FPS starts every distance at numeric_limits::max(), never
// re-selects a point and takes degenerate points first).
//
// Unlike the reference's single-threaded loops they run on at::parallel_for,
// split only where the result cannot depend on the split:
//   - KNN forward: independent query rows;
//   - KNN backward: grad_p1 by query rows; grad_p2 by ranges of destination
//     points, each range applying its updates in the reference's (row, slot)
//     order, so every element sees the same sequence of roundings;
//   - FPS: clouds in parallel, or, for few clouds, chunks of one cloud's
//     points whose per-chunk maxima are combined in chunk order (the first
//     index of the greatest distance, as the sequential scan finds it);
//   - gather: (cloud, channel) rows, the backward's duplicates summed in
//     sample order within each row.
// Lengths outside [0, P] are clamped and indices outside the cloud are
// skipped (gather forward: 0); the reference reads out of bounds there.
#include <torch/all.h>
#include <torch/library.h>

#include <ATen/Parallel.h>

#include <algorithm>
#include <cmath>
#include <limits>
#include <utility>
#include <vector>

namespace torch_point_ops {
namespace {

template <typename T>
inline T abs_of(T v) {
  return v < T(0) ? T(-v) : v;
}
template <>
inline c10::Half abs_of(c10::Half v) {
  return c10::Half(std::fabs(static_cast<float>(v)));
}

inline int64_t clamp_len(int64_t v, int64_t hi) { return v < 0 ? 0 : (v > hi ? hi : v); }

void check_cpu_floating(const at::Tensor& t, const char* op) {
  const auto st = t.scalar_type();
  TORCH_CHECK(st == at::kFloat || st == at::kDouble || st == at::kHalf, "\"", op,
              "\" not implemented for '", st, "'");
}

// ---------------------------------------------------------------- knn
// One query row: the K smallest (dist, index) pairs of p2[0:l2] under the
// order of std::tuple<scalar_t,int> (knn.cpp:60), kept in a max-heap with
// the same pushes and pops as the reference's std::priority_queue, then
// emptied in ascending order (std::sort_heap performs the same sequence of
// pop_heap steps as repeated top()/pop()).
template <typename T>
void knn_row(const T* q, const T* p2, int64_t l2, int64_t D, int64_t K, int norm,
             std::vector<std::pair<T, int>>& heap, int64_t* idx_out, T* dist_out) {
  heap.clear();
  for (int64_t j = 0; j < l2; ++j) {
    const T* r = p2 + j * D;
    T dist = T(0);
    if (norm == 1) {
      for (int64_t d = 0; d < D; ++d) dist += abs_of<T>(T(q[d] - r[d]));
    } else {
      for (int64_t d = 0; d < D; ++d) {
        const T diff = q[d] - r[d];
        dist += T(diff * diff);
      }
    }
    if ((int64_t)heap.size() < K || dist < heap.front().first) {
      heap.emplace_back(dist, (int)j);
      std::push_heap(heap.begin(), heap.end());
      if ((int64_t)heap.size() > K) {
        std::pop_heap(heap.begin(), heap.end());
        heap.pop_back();
      }
    }
  }
  std::sort_heap(heap.begin(), heap.end());
  for (size_t k = 0; k < heap.size(); ++k) {
    dist_out[k] = heap[k].first;
    idx_out[k] = heap[k].second;
  }
}

template <typename T>
void knn_forward_cpu_impl(const at::Tensor& p1, const at::Tensor& p2, const int64_t* l1,
                          const int64_t* l2, int64_t K, int norm, at::Tensor& idxs,
                          at::Tensor& dists) {
  const int64_t N = p1.size(0), P1 = p1.size(1), P2 = p2.size(1), D = p1.size(2);
  const T* a = p1.data_ptr<T>();
  const T* b = p2.data_ptr<T>();
  int64_t* io = idxs.data_ptr<int64_t>();
  T* dout = dists.data_ptr<T>();
  // grain: about 2^16 distance evaluations per task
  const int64_t grain = std::max<int64_t>(1, (int64_t)65536 / std::max<int64_t>(1, P2 * D));
  at::parallel_for(0, N * P1, grain, [&](int64_t begin, int64_t end) {
    std::vector<std::pair<T, int>> heap;
    heap.reserve((size_t)K + 1);
    for (int64_t row = begin; row < end; ++row) {
      const int64_t n = row / P1, i = row - n * P1;
      if (i >= clamp_len(l1[n], P1)) continue;
      knn_row<T>(a + row * D, b + n * P2 * D, clamp_len(l2[n], P2), D, K, norm, heap,
                 io + row * K, dout + row * K);
    }
  });
}

std::tuple<at::Tensor, at::Tensor> knn_forward_cpu(const at::Tensor& p1_in,
                                                   const at::Tensor& p2_in,
                                                   const at::Tensor& lengths1_in,
                                                   const at::Tensor& lengths2_in, int64_t norm,
                                                   int64_t K, int64_t version) {
  (void)version;  // the reference's CPU kernel has one implementation
  TORCH_CHECK(p1_in.dim() == 3 && p2_in.dim() == 3, "knn_forward expects (N,P,D) tensors");
  TORCH_CHECK(lengths1_in.scalar_type() == at::kLong && lengths2_in.scalar_type() == at::kLong,
              "lengths must be int64");
  TORCH_CHECK((norm == 1) || (norm == 2), "Norm must be 1 or 2.");
  TORCH_CHECK(K >= 0, "K must be non-negative");
  const int64_t N = p1_in.size(0), P1 = p1_in.size(1), D = p1_in.size(2);
  // knn.cpp:43-45: idxs start at -1, dists at 0
  at::Tensor idxs = at::full({N, P1, K}, -1, lengths1_in.options().dtype(at::kLong));
  at::Tensor dists = at::zeros({N, P1, K}, p1_in.options());
  check_cpu_floating(p1_in, "knn_cpu_forward");
  if (idxs.numel() == 0) return {idxs, dists};
  TORCH_CHECK(p2_in.size(0) == N && lengths1_in.numel() == N && lengths2_in.numel() == N,
              "batch sizes differ");
  TORCH_CHECK(p2_in.size(2) == D, "Point sets must have the same last dimension");
  TORCH_CHECK(p1_in.scalar_type() == p2_in.scalar_type(), "p1 and p2 dtypes differ");
  TORCH_CHECK(K < std::numeric_limits<int>::max() && p2_in.size(1) < std::numeric_limits<int>::max(),
              "knn_forward: sizes too large for the CPU kernel");
  const at::Tensor p1 = p1_in.contiguous(), p2 = p2_in.contiguous();
  const at::Tensor l1 = lengths1_in.contiguous(), l2 = lengths2_in.contiguous();
  switch (p1.scalar_type()) {
    case at::kFloat:
      knn_forward_cpu_impl<float>(p1, p2, l1.data_ptr<int64_t>(), l2.data_ptr<int64_t>(), K,
                                  (int)norm, idxs, dists);
      break;
    case at::kDouble:
      knn_forward_cpu_impl<double>(p1, p2, l1.data_ptr<int64_t>(), l2.data_ptr<int64_t>(), K,
                                   (int)norm, idxs, dists);
      break;
    default:
      knn_forward_cpu_impl<c10::Half>(p1, p2, l1.data_ptr<int64_t>(), l2.data_ptr<int64_t>(), K,
                                      (int)norm, idxs, dists);
      break;
  }
  return {idxs, dists};
}

// The reference's per-coordinate gradient term (knn.cpp:146-156):
// L1: g * (p1 > p2 ? 1 : -1); L2: 2.0 * g * (p1 - p2) with the product in
// double (2.0 is a double literal), stored to T with one rounding.
template <typename T>
inline T knn_grad_term(T g, T v1, T v2, int norm) {
  if (norm == 1) return g * ((v1 > v2) ? T(1.0) : T(-1.0));
  return static_cast<T>(2.0 * g * (v1 - v2));
}
template <>
inline c10::Half knn_grad_term(c10::Half g, c10::Half v1, c10::Half v2, int norm) {
  if (norm == 1) return g * ((v1 > v2) ? c10::Half(1.0f) : c10::Half(-1.0f));
  const double t = 2.0 * g * c10::Half(v1 - v2);  // c10 operator*(double, Half) -> double
  return c10::Half(static_cast<float>(t));        // Half(double) converts through float
}

template <typename T>
void knn_backward_cpu_impl(const at::Tensor& p1, const at::Tensor& p2, const int64_t* len1,
                           const int64_t* len2, const at::Tensor& idxs, int norm,
                           const at::Tensor& gd, at::Tensor& g1, at::Tensor& g2) {
  const int64_t N = p1.size(0), P1 = p1.size(1), P2 = p2.size(1), D = p1.size(2);
  const int64_t K = idxs.size(2);
  const T* a = p1.data_ptr<T>();
  const T* b = p2.data_ptr<T>();
  const int64_t* ix = idxs.data_ptr<int64_t>();
  const T* g = gd.data_ptr<T>();
  T* o1 = g1.data_ptr<T>();
  T* o2 = g2.data_ptr<T>();
  // slots k < min(lengths2, K) of rows i < lengths1 (knn.cpp:137-141)
  auto slots = [&](int64_t n) { return std::min<int64_t>(std::max<int64_t>(len2[n], 0), K); };
  // grad_p1: each row sums its own slots in slot order
  at::parallel_for(0, N * P1, std::max<int64_t>(1, 4096 / std::max<int64_t>(1, K * D)),
                   [&](int64_t begin, int64_t end) {
                     for (int64_t row = begin; row < end; ++row) {
                       const int64_t n = row / P1, i = row - n * P1;
                       if (i >= clamp_len(len1[n], P1)) continue;
                       const int64_t ks = slots(n);
                       for (int64_t k = 0; k < ks; ++k) {
                         const int64_t j = ix[row * K + k];
                         if (j < 0 || j >= P2) continue;  // -1 padding (and out of range)
                         for (int64_t d = 0; d < D; ++d)
                           o1[row * D + d] += knn_grad_term<T>(g[row * K + k], a[row * D + d],
                                                               b[(n * P2 + j) * D + d], norm);
                       }
                     }
                   });
  // grad_p2: split every cloud's points into ranges; a range walks all
  // (row, slot) pairs of its cloud in order and applies the ones landing in it
  const int64_t chunk = std::max<int64_t>(256, (P2 + 15) / 16);
  const int64_t per = (P2 + chunk - 1) / chunk;
  at::parallel_for(0, N * per, 1, [&](int64_t begin, int64_t end) {
    for (int64_t t = begin; t < end; ++t) {
      const int64_t n = t / per, lo = (t - n * per) * chunk, hi = std::min(lo + chunk, P2);
      const int64_t l1 = clamp_len(len1[n], P1), ks = slots(n);
      for (int64_t i = 0; i < l1; ++i) {
        const int64_t row = n * P1 + i;
        for (int64_t k = 0; k < ks; ++k) {
          const int64_t j = ix[row * K + k];
          if (j < lo || j >= hi) continue;
          for (int64_t d = 0; d < D; ++d)
            o2[(n * P2 + j) * D + d] -= knn_grad_term<T>(g[row * K + k], a[row * D + d],
                                                         b[(n * P2 + j) * D + d], norm);
        }
      }
    }
  });
}

std::tuple<at::Tensor, at::Tensor> knn_backward_cpu(const at::Tensor& p1_in,
                                                    const at::Tensor& p2_in,
                                                    const at::Tensor& lengths1_in,
                                                    const at::Tensor& lengths2_in,
                                                    const at::Tensor& idxs_in, int64_t norm,
                                                    const at::Tensor& grad_dists_in) {
  TORCH_CHECK(p1_in.dim() == 3 && p2_in.dim() == 3 && idxs_in.dim() == 3,
              "knn_backward expects (N,P,D) points and (N,P1,K) idxs");
  const int64_t N = p1_in.size(0), P1 = p1_in.size(1), D = p1_in.size(2);
  TORCH_CHECK(p2_in.size(0) == N && p2_in.size(2) == D, "Point sets must have the same last dimension");
  TORCH_CHECK(idxs_in.size(0) == N && idxs_in.size(1) == P1, "idxs shape differs from p1");
  TORCH_CHECK(grad_dists_in.sizes() == idxs_in.sizes(), "grad_dists shape differs from idxs");
  TORCH_CHECK(idxs_in.scalar_type() == at::kLong && lengths1_in.scalar_type() == at::kLong &&
                  lengths2_in.scalar_type() == at::kLong,
              "idxs and lengths must be int64");
  TORCH_CHECK(lengths1_in.numel() == N && lengths2_in.numel() == N, "batch sizes differ");
  TORCH_CHECK((norm == 1) || (norm == 2), "Norm must be 1 or 2.");
  check_cpu_floating(p1_in, "knn_cpu_backward");
  TORCH_CHECK(p2_in.scalar_type() == p1_in.scalar_type() &&
                  grad_dists_in.scalar_type() == p1_in.scalar_type(),
              "p1, p2 and grad_dists dtypes differ");
  const at::Tensor p1 = p1_in.contiguous(), p2 = p2_in.contiguous();
  const at::Tensor l1 = lengths1_in.contiguous(), l2 = lengths2_in.contiguous();
  const at::Tensor idxs = idxs_in.contiguous(), gd = grad_dists_in.contiguous();
  at::Tensor g1 = at::zeros(p1.sizes(), p1.options());
  at::Tensor g2 = at::zeros(p2.sizes(), p2.options());
  if (g1.numel() == 0 || g2.numel() == 0 || idxs.numel() == 0) return {g1, g2};
  switch (p1.scalar_type()) {
    case at::kFloat:
      knn_backward_cpu_impl<float>(p1, p2, l1.data_ptr<int64_t>(), l2.data_ptr<int64_t>(), idxs,
                                   (int)norm, gd, g1, g2);
      break;
    case at::kDouble:
      knn_backward_cpu_impl<double>(p1, p2, l1.data_ptr<int64_t>(), l2.data_ptr<int64_t>(), idxs,
                                    (int)norm, gd, g1, g2);
      break;
    default:
      knn_backward_cpu_impl<c10::Half>(p1, p2, l1.data_ptr<int64_t>(), l2.data_ptr<int64_t>(),
                                       idxs, (int)norm, gd, g1, g2);
      break;
  }
  return {g1, g2};
}

// ---------------------------------------------------------------- fps
// A cloud's state between iterations: the running minimum of every point
// and whether it was selected.  A point takes part in the update only when
// it is unselected and x*x + y*y + z*z is not <= scalar_t(1e-3)
// (fps.cpp:53-58); that test does not change between iterations, so it is
// made once.
template <typename T>
struct FpsCloud {
  const T* p;
  int64_t n;
  std::vector<T> md;
  std::vector<uint8_t> live;  // unselected
  std::vector<uint8_t> upd;   // takes part in the distance update

  FpsCloud(const T* pts, int64_t count) : p(pts), n(count), md(count), live(count, 1), upd(count) {
    const T thr = T(1e-3);
    for (int64_t j = 0; j < n; ++j) {
      const T x = p[3 * j], y = p[3 * j + 1], z = p[3 * j + 2];
      const T mag = T(T(x * x) + T(y * y)) + T(z * z);
      upd[j] = !(mag <= thr);
      md[j] = std::numeric_limits<T>::max();
    }
  }

  // update [lo, hi) against the sample c; return the first index of the
  // strictly greatest running minimum among the live points (-1: none)
  std::pair<T, int64_t> sweep(int64_t lo, int64_t hi, T cx, T cy, T cz) {
    T best = T(-1);
    int64_t bi = -1;
    for (int64_t j = lo; j < hi; ++j) {
      if (!live[j]) continue;
      if (upd[j]) {
        const T dx = p[3 * j] - cx, dy = p[3 * j + 1] - cy, dz = p[3 * j + 2] - cz;
        const T dist = T(T(dx * dx) + T(dy * dy)) + T(dz * dz);
        md[j] = std::min(md[j], dist);
      }
      if (md[j] > best) {
        best = md[j];
        bi = j;
      }
    }
    return {best, bi};
  }
};

// Running minima are never NaN: std::min keeps the old value unless the new
// distance is strictly smaller, and they start finite.  So the sequential
// scan's winner (first index whose value beats every earlier one) is the
// first index attaining the maximum, and chunk winners combine by value,
// then by chunk order.
template <typename T>
void fps_cloud(const T* pts, int64_t n, int64_t m, int64_t* out, int64_t nchunks) {
  FpsCloud<T> c(pts, n);
  int64_t cur = 0;
  out[0] = 0;
  c.live[0] = 0;
  const int64_t chunk = (n + nchunks - 1) / nchunks;
  std::vector<std::pair<T, int64_t>> part((size_t)nchunks);
  for (int64_t i = 1; i < m; ++i) {
    const T cx = pts[3 * cur], cy = pts[3 * cur + 1], cz = pts[3 * cur + 2];
    if (nchunks == 1) {
      part[0] = c.sweep(0, n, cx, cy, cz);
    } else {
      at::parallel_for(0, nchunks, 1, [&](int64_t b, int64_t e) {
        for (int64_t t = b; t < e; ++t)
          part[t] = c.sweep(std::min(t * chunk, n), std::min((t + 1) * chunk, n), cx, cy, cz);
      });
    }
    T best = T(-1);
    int64_t bi = 0;  // fps.cpp:73: index 0 when no point is left
    for (int64_t t = 0; t < nchunks; ++t)
      if (part[t].second >= 0 && part[t].first > best) {
        best = part[t].first;
        bi = part[t].second;
      }
    cur = bi;
    out[i] = cur;
    c.live[cur] = 0;
  }
}

template <typename T>
void fps_cpu_impl(const at::Tensor& points, int64_t m, at::Tensor& idx) {
  const int64_t B = points.size(0), n = points.size(1);
  const T* p = points.data_ptr<T>();
  int64_t* o = idx.data_ptr<int64_t>();
  const int64_t threads = at::get_num_threads();
  if (B >= threads || n < 8192) {
    at::parallel_for(0, B, 1, [&](int64_t b0, int64_t b1) {
      for (int64_t b = b0; b < b1; ++b) fps_cloud<T>(p + b * n * 3, n, m, o + b * m, 1);
    });
  } else {
    const int64_t nchunks = std::min<int64_t>(threads, n / 4096);
    for (int64_t b = 0; b < B; ++b) fps_cloud<T>(p + b * n * 3, n, m, o + b * m, nchunks);
  }
}

at::Tensor fps_forward_cpu(const at::Tensor& points_in, int64_t nsamples) {
  TORCH_CHECK(points_in.dim() == 3, "fps_forward expects (N,P,3)");
  const int64_t P = points_in.size(1), D = points_in.size(2);
  // fps.cpp:23-25
  TORCH_CHECK(D == 3, "FPS only supports 3D points, but got dimension ", D);
  TORCH_CHECK(nsamples > 0, "nsamples must be positive, but got ", nsamples);
  TORCH_CHECK(nsamples <= P, "nsamples (", nsamples, ") cannot exceed number of points (", P,
              ")");
  at::Tensor idx = at::zeros({points_in.size(0), nsamples}, at::kLong);
  check_cpu_floating(points_in, "fps_cpu_forward");
  if (idx.numel() == 0) return idx;
  const at::Tensor points = points_in.contiguous();
  switch (points.scalar_type()) {
    case at::kFloat: fps_cpu_impl<float>(points, nsamples, idx); break;
    case at::kDouble: fps_cpu_impl<double>(points, nsamples, idx); break;
    default: fps_cpu_impl<c10::Half>(points, nsamples, idx); break;
  }
  return idx;
}

// fps.cpp:144-155: the CPU path ignores kd_depth after checking it
at::Tensor quick_fps_forward_cpu(const at::Tensor& points, int64_t nsamples, int64_t kd_depth) {
  TORCH_CHECK(points.dim() == 3, "quick_fps_forward expects (N,P,3)");
  const int64_t P = points.size(1), D = points.size(2);
  TORCH_CHECK(D == 3, "Quick FPS only supports 3D points, but got dimension ", D);
  TORCH_CHECK(nsamples > 0, "nsamples must be positive, but got ", nsamples);
  TORCH_CHECK(nsamples <= P, "nsamples (", nsamples, ") cannot exceed number of points (", P,
              ")");
  TORCH_CHECK(kd_depth > 0 && kd_depth <= 10, "kd_depth must be between 1 and 10, but got ",
              kd_depth);
  return fps_forward_cpu(points, nsamples);
}

// ------------------------------------------------------------- gather
template <typename T>
void gather_fwd_cpu_impl(const at::Tensor& pts, const at::Tensor& idx, at::Tensor& out) {
  const int64_t B = pts.size(0), C = pts.size(1), N = pts.size(2), M = idx.size(1);
  const T* p = pts.data_ptr<T>();
  const int64_t* ix = idx.data_ptr<int64_t>();
  T* o = out.data_ptr<T>();
  at::parallel_for(0, B * C, std::max<int64_t>(1, 16384 / std::max<int64_t>(1, M)),
                   [&](int64_t r0, int64_t r1) {
                     for (int64_t r = r0; r < r1; ++r) {
                       const int64_t b = r / C;
                       const T* src = p + r * N;
                       for (int64_t j = 0; j < M; ++j) {
                         const int64_t a = ix[b * M + j];
                         o[r * M + j] = (a >= 0 && a < N) ? src[a] : T(0);
                       }
                     }
                   });
}

template <typename T>
void gather_bwd_cpu_impl(const at::Tensor& go, const at::Tensor& idx, int64_t N, at::Tensor& gp) {
  const int64_t B = go.size(0), C = go.size(1), M = go.size(2);
  const T* g = go.data_ptr<T>();
  const int64_t* ix = idx.data_ptr<int64_t>();
  T* o = gp.data_ptr<T>();
  at::parallel_for(0, B * C, std::max<int64_t>(1, 16384 / std::max<int64_t>(1, M)),
                   [&](int64_t r0, int64_t r1) {
                     for (int64_t r = r0; r < r1; ++r) {
                       const int64_t b = r / C;
                       T* dst = o + r * N;
                       for (int64_t j = 0; j < M; ++j) {
                         const int64_t a = ix[b * M + j];
                         if (a >= 0 && a < N) dst[a] += g[r * M + j];
                       }
                     }
                   });
}

at::Tensor gather_points_forward_cpu(const at::Tensor& points_in, const at::Tensor& idx_in) {
  TORCH_CHECK(points_in.dim() == 3 && idx_in.dim() == 2, "gather_points expects (N,C,P), (N,M)");
  TORCH_CHECK(idx_in.scalar_type() == at::kLong, "gather_points expects int64 indices");
  TORCH_CHECK(idx_in.size(0) == points_in.size(0), "batch sizes differ");
  check_cpu_floating(points_in, "gather_points_cpu_forward");
  at::Tensor out = at::zeros({points_in.size(0), points_in.size(1), idx_in.size(1)},
                             points_in.options());
  if (out.numel() == 0) return out;
  const at::Tensor points = points_in.contiguous(), idx = idx_in.contiguous();
  switch (points.scalar_type()) {
    case at::kFloat: gather_fwd_cpu_impl<float>(points, idx, out); break;
    case at::kDouble: gather_fwd_cpu_impl<double>(points, idx, out); break;
    default: gather_fwd_cpu_impl<c10::Half>(points, idx, out); break;
  }
  return out;
}

at::Tensor gather_points_backward_cpu(const at::Tensor& grad_in, const at::Tensor& idx_in,
                                      int64_t n) {
  TORCH_CHECK(grad_in.dim() == 3 && idx_in.dim() == 2, "gather_points_backward expects 3D/2D");
  TORCH_CHECK(idx_in.scalar_type() == at::kLong, "gather_points expects int64 indices");
  TORCH_CHECK(n >= 0, "n must be non-negative");
  TORCH_CHECK(idx_in.size(0) == grad_in.size(0) && idx_in.size(1) == grad_in.size(2),
              "idx shape differs from grad_out");
  check_cpu_floating(grad_in, "gather_points_cpu_backward");
  at::Tensor out = at::zeros({grad_in.size(0), grad_in.size(1), n}, grad_in.options());
  if (out.numel() == 0) return out;
  const at::Tensor go = grad_in.contiguous(), idx = idx_in.contiguous();
  switch (go.scalar_type()) {
    case at::kFloat: gather_bwd_cpu_impl<float>(go, idx, n, out); break;
    case at::kDouble: gather_bwd_cpu_impl<double>(go, idx, n, out); break;
    default: gather_bwd_cpu_impl<c10::Half>(go, idx, n, out); break;
  }
  return out;
}

}  // namespace

TORCH_LIBRARY_IMPL(torch_point_ops_knn, CPU, m) {
  m.impl("knn_forward", &knn_forward_cpu);
  m.impl("knn_backward", &knn_backward_cpu);
}

TORCH_LIBRARY_IMPL(torch_point_ops_fps, CPU, m) {
  m.impl("fps_forward", &fps_forward_cpu);
  m.impl("gather_points_forward", &gather_points_forward_cpu);
  m.impl("gather_points_backward", &gather_points_backward_cpu);
}

TORCH_LIBRARY_IMPL(torch_point_ops_quick_fps, CPU, m) {
  m.impl("quick_fps_forward", &quick_fps_forward_cpu);
}

}  // namespace torch_point_ops
