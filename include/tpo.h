/*
 * tpo.h -- C ABI of libtpo_hip.so, the MI355X (gfx950) kernels behind the
 * torch_point_ops operators chamfer / knn / fps / gather_points / emd.
 *
 * Conventions for every entry point:
 *   - all pointers are device pointers (hipMalloc / torch CUDA-device tensors)
 *     to contiguous row-major arrays; `stream` is a hipStream_t (or NULL for
 *     the default stream) and every call is asynchronous on it;
 *   - no entry point allocates, frees or synchronises; buffers that need
 *     scratch take a caller-provided workspace sized by a *_workspace_size()
 *     query;
 *   - outputs are written completely (no pre-zeroing needed);
 *   - return 0 on success or a negative TPO_ERR_* code; tpo_last_error()
 *     returns a thread-local description of the last failure;
 *   - dtype is one of TPO_F32, TPO_F64, TPO_F16 (IEEE binary16), TPO_BF16
 *     (only where stated).
 * The functions keep no global mutable state (apart from
 * tpo_chamfer_fwd_noalloc's static device scratch and its per-device address
 * cache) and may be called from any thread.
 */
#ifndef TPO_H
#define TPO_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  TPO_F32 = 0,
  TPO_F64 = 1,
  TPO_F16 = 2,
  TPO_BF16 = 3
};

enum {
  TPO_OK = 0,
  TPO_ERR_ARG = -1,       /* bad size / argument */
  TPO_ERR_DTYPE = -2,     /* dtype not supported by this entry point */
  TPO_ERR_LAUNCH = -3,    /* HIP launch error (message from hipGetLastError) */
  TPO_ERR_WORKSPACE = -4  /* workspace missing or too small */
};

/* Thread-local message for the last non-zero return on this thread. */
const char* tpo_last_error(void);

/* ABI version of this header (major << 16 | minor). */
int tpo_abi_version(void);

/*
 * Chamfer forward.  Replaces chamfer_cuda_forward
 * (torch_point_ops/chamfer/csrc/cuda/chamfer.cu:169-198), the CUDA-key body
 * of torch_point_ops_chamfer::chamfer_forward (chamfer.cpp:35-36).
 *   xyz1 (B,N,3), xyz2 (B,M,3) of `dtype` (F32/F64/F16)
 *   dist1 (B,N), dist2 (B,M) of `dtype`: squared distance to the nearest
 *   point of the other cloud; idx1 (B,N), idx2 (B,M) int32: the FIRST index
 *   attaining it.  An empty other cloud gives dist 0, idx 0.
 *   workspace (optional, tpo_chamfer_workspace_size() bytes, 256-byte
 *   aligned; size 0 means none is used): with it, float and half clouds of
 *   at least 2048 points each are searched with exact spatial pruning, which
 *   is much faster on clustered or spread-out data; results are identical
 *   with or without it.
 */
int64_t tpo_chamfer_workspace_size(int dtype, int64_t B, int64_t N, int64_t M);
int tpo_chamfer_fwd(int dtype, const void* xyz1, const void* xyz2,
                    int64_t B, int64_t N, int64_t M,
                    void* dist1, void* dist2, int32_t* idx1, int32_t* idx2,
                    void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Chamfer forward that allocates nothing.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory or pass a workspace
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as tpo_chamfer_fwd, bit for bit;
 * the grid-search workspace is a static device array of
 * tpo_chamfer_noalloc_max_workspace() bytes (32 MiB) that every GPU the
 * library runs on holds until the process ends.  Sizes whose workspace
 * (tpo_chamfer_workspace_size) exceeds it are rejected with
 * TPO_ERR_WORKSPACE (B=32, N=M=8192 needs about 19 MB).  All calls on one
 * device share that array: calls that overlap on one GPU (other streams or
 * threads) race; calls ordered on one stream do not.
 */
int64_t tpo_chamfer_noalloc_max_workspace(void);
int tpo_chamfer_fwd_noalloc(int dtype, const void* xyz1, const void* xyz2,
                            int64_t B, int64_t N, int64_t M,
                            void* dist1, void* dist2, int32_t* idx1, int32_t* idx2,
                            void* stream);

/*
 * Diagnostic, no counterpart in the reference: after a tpo_chamfer_fwd call
 * that used the workspace (same dtype and sizes), writes to the device
 * int64 `pairs` the number of (query, reference) pairs the pruned search
 * evaluated (a brute-force search evaluates 2*B*N*M).  Asynchronous on
 * `stream`.
 */
int tpo_chamfer_pairs_evaluated(int dtype, const void* workspace, int64_t B,
                                int64_t N, int64_t M, int64_t* pairs, void* stream);

/*
 * Chamfer backward.  Replaces chamfer_cuda_backward (chamfer.cu:236-271),
 * torch_point_ops_chamfer::chamfer_backward (chamfer.cpp:37-38).
 *   grad_dist1 (B,N), grad_dist2 (B,M) of `dtype`
 *   grad_xyz1 (B,N,3), grad_xyz2 (B,M,3) of `dtype`:
 *     grad_xyz1[i] =  2 g1[i] (x1_i - x2_idx1[i]) - sum_{j: idx2[j]=i} 2 g2[j] (x2_j - x1_i)
 *   (and symmetrically), the scatter summed by atomics in unspecified order.
 */
int tpo_chamfer_bwd(int dtype, const void* xyz1, const void* xyz2,
                    const int32_t* idx1, const int32_t* idx2,
                    const void* grad_dist1, const void* grad_dist2,
                    int64_t B, int64_t N, int64_t M,
                    void* grad_xyz1, void* grad_xyz2, void* stream);

/*
 * Chamfer loss: ChamferDistance(reduction="mean" / "sum")
 * (torch_point_ops/chamfer/chamfer.py:18-24) in one forward and one
 * backward call.  No single counterpart in the reference, which reduces
 * chamfer_forward's distances with torch.mean / torch.sum; these entry points
 * fuse that reduction into the forward and the reduction's gradient into the
 * backward.
 *   loss (one element of `dtype`): mean != 0: mean(dist1) + mean(dist2)
 *     (NaN when a cloud is empty, like torch.mean); mean == 0: sum + sum.
 *     The sums are taken in a fixed order, so the loss is deterministic; it
 *     matches torch's reduction of tpo_chamfer_fwd's distances to rounding.
 *   idx1, idx2 as tpo_chamfer_fwd (the backward needs them); the distances
 *   themselves are not stored.
 *   workspace (required): tpo_chamfer_loss_workspace_size() bytes, 256-byte
 *   aligned, contents need not be initialised.
 * tpo_chamfer_loss_bwd: grad_loss is ONE device element of `dtype`; the
 *   gradients equal tpo_chamfer_bwd's with grad_dist = grad_loss / numel
 *   (mean, multiplied by the reciprocal as torch's MeanBackward does) or
 *   grad_loss (sum) for every point.
 */
int64_t tpo_chamfer_loss_workspace_size(int dtype, int64_t B, int64_t N, int64_t M);
int tpo_chamfer_loss_fwd(int dtype, const void* xyz1, const void* xyz2,
                         int64_t B, int64_t N, int64_t M, int mean, void* loss,
                         int32_t* idx1, int32_t* idx2,
                         void* workspace, int64_t workspace_bytes, void* stream);
int tpo_chamfer_loss_bwd(int dtype, const void* xyz1, const void* xyz2,
                         const int32_t* idx1, const int32_t* idx2,
                         const void* grad_loss, int mean,
                         int64_t B, int64_t N, int64_t M,
                         void* grad_xyz1, void* grad_xyz2, void* stream);

/*
 * KNN forward.  Replaces knn_cuda_forward
 * (torch_point_ops/knn/csrc/cuda/knn.cu:295-398),
 * torch_point_ops_knn::knn_forward (knn.cpp:168-169).
 *   p1 (N,P1,D), p2 (N,P2,D) of `dtype`; lengths1/lengths2 (N) int64
 *   (clamped to [0,P1] / [0,P2]); norm 1 or 2; K >= 1; version -1 for
 *   automatic, 0..3 to force one of the reference's kernel semantics (an
 *   invalid choice falls back to automatic, as the reference does).
 *   F32/F64/F16: idxs (N,P1,K) int64 and dists (N,P1,K) `dtype`, unsorted,
 *   laid out exactly as the reference's MinK slots, including its padding
 *   rules: rows >= lengths1 are (0,0); slots >= lengths2 are (0,0) for
 *   versions 2/3 and (-1,+inf) for versions 0/1.  workspace is optional
 *   (tpo_knn_workspace_size bytes): with it the queries are processed in
 *   spatial order, which is faster; results are identical.
 *   BF16 (no reference kernel; the reference raises): norm 2, D % 8 == 0,
 *   8 <= D <= 128, K <= 32, points 16-byte aligned, workspace required.
 *   Squared distances |q|^2 + |r|^2 - 2 q.r in float, summed on the matrix
 *   cores (the norms, float sums of the bf16 squares, enter as exact
 *   three-piece bf16 splits), clamped at 0; each row's K nearest sorted by
 *   (distance, index), dists rounded to bfloat16; rows >= lengths1 and
 *   slots >= lengths2 are (0,0).  version is ignored and version_out
 *   receives -1.  For P2 >= max(4096, 1536 K) the workspace also holds a
 *   per-query bound sampled from 64 tiles of 32 references, the candidates
 *   at or below it (up to 128 per query and reference slice) and a list of
 *   the rows that overflowed or fell short (and every row of a cloud whose
 *   lengths2 is below that size), which are recomputed without it; results
 *   do not depend on it.
 *   If version_out is not NULL it receives the version that ran.
 */
int64_t tpo_knn_workspace_size(int dtype, int64_t N, int64_t P1, int64_t P2,
                               int64_t D, int64_t K, int norm);
int tpo_knn_fwd(int dtype, const void* p1, const void* p2,
                const int64_t* lengths1, const int64_t* lengths2,
                int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K,
                int norm, int version, int64_t* idxs, void* dists,
                int* version_out, void* workspace, int64_t workspace_bytes,
                void* stream);

/*
 * KNN forward with the rows sorted the way knn_points(return_sorted=True)
 * returns them (torch_point_ops/knn/__init__.py:111-131: torch's sort of
 * each row after the forward, slots past lengths2 keyed +inf, then zeroed).
 * No single counterpart in the reference: the forward and the module's sort
 * in one launch.  F32/F64/F16 with 2 <= K <= 32 only; arguments and padding
 * as tpo_knn_fwd.  Each row is sorted by replaying torch's 32-wide bitonic
 * network, so equal distances come out in the same order as torch.sort
 * puts them.
 */
int tpo_knn_fwd_sorted(int dtype, const void* p1, const void* p2,
                       const int64_t* lengths1, const int64_t* lengths2,
                       int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K,
                       int norm, int version, int64_t* idxs, void* dists,
                       int* version_out, void* workspace, int64_t workspace_bytes,
                       void* stream);

/*
 * knn_gather forward.  Replaces the expand + gather + mask of
 * knn_gather (torch_point_ops/knn/__init__.py:136-183), which the reference
 * runs as torch ops.
 *   x (N,M,U), idx (N,L,K) int64, lengths (N) int64 valid counts of x;
 *   out (N,L,K,U) of `dtype` (F32/F64/F16/BF16): out[n,l,k] = x[n, idx[n,l,k]]
 *   for k < lengths[n], else 0 (and 0 for an index outside [0, M)).
 */
int tpo_knn_gather(int dtype, const void* x, const int64_t* idx,
                   const int64_t* lengths, int64_t N, int64_t M, int64_t L, int64_t K,
                   int64_t U, void* out, void* stream);

/*
 * KNN backward.  Replaces knn_cuda_backward (knn.cu:469-534),
 * torch_point_ops_knn::knn_backward (knn.cpp:170-171).
 *   idxs / grad_dists (N,P1,K); grad_p1 (N,P1,D), grad_p2 (N,P2,D) `dtype`.
 *   Rows >= lengths1 and slots with idx == -1 contribute nothing; L2:
 *   diff = (2 g)(p1 - p2); L1: diff = g sign(p1 - p2) with sign(0) = 0;
 *   grad_p1 += diff, grad_p2[idx] -= diff.
 */
int tpo_knn_bwd(int dtype, const void* p1, const void* p2,
                const int64_t* lengths1, const int64_t* lengths2,
                const int64_t* idxs, int norm, const void* grad_dists,
                int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K,
                void* grad_p1, void* grad_p2, void* stream);

/*
 * tpo_knn_bwd with a workspace (the same reference function,
 * knn_cuda_backward, knn.cu:469-534).  With workspace_bytes >=
 * tpo_knn_bwd_workspace_size() (non-zero for D <= 7, K <= 256 and
 * reference clouds up to ~750 K points) grad_p2 is accumulated without
 * global atomics: the terms are grouped by reference rows in the workspace
 * and each group is summed in LDS.  A smaller or NULL workspace runs the
 * atomic scatter of tpo_knn_bwd.  workspace: 256-byte aligned.
 */
int64_t tpo_knn_bwd_workspace_size(int dtype, int64_t N, int64_t P1, int64_t P2, int64_t D,
                                   int64_t K);
int tpo_knn_bwd_ws(int dtype, const void* p1, const void* p2,
                   const int64_t* lengths1, const int64_t* lengths2,
                   const int64_t* idxs, int norm, const void* grad_dists,
                   int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K,
                   void* grad_p1, void* grad_p2, void* workspace, int64_t workspace_bytes,
                   void* stream);

/*
 * Furthest point sampling.  Replaces fps_cuda_forward
 * (torch_point_ops/fps/csrc/cuda/fps.cu:273-315),
 * torch_point_ops_fps::fps_forward (fps.cpp:159).
 *   points (B,N,3) `dtype` (F32/F64/F16), 1 <= nsamples <= N;
 *   idx (B,nsamples) int64, identical to the reference kernel including its
 *   skip rule (|p|^2 <= 1e-3 never selected), start index 0 and tie order.
 *   workspace: tpo_fps_workspace_size(dtype, B, N) bytes, 256-byte aligned.
 */
int64_t tpo_fps_workspace_size(int dtype, int64_t B, int64_t N);
int tpo_fps_fwd(int dtype, const void* points, int64_t B, int64_t N,
                int64_t nsamples, int64_t* idx,
                void* workspace, int64_t workspace_bytes, void* stream);

/*
 * gather_points forward.  Replaces gather_points_cuda_forward
 * (fps.cu:318-357), torch_point_ops_fps::gather_points_forward (fps.cpp:160).
 *   points (B,C,N), idx (B,M) int64 in [0,N), out (B,C,M).  F32/F64/F16.
 */
int tpo_gather_fwd(int dtype, const void* points, const int64_t* idx,
                   int64_t B, int64_t C, int64_t N, int64_t M, void* out,
                   void* stream);

/*
 * gather_points backward.  Replaces gather_points_cuda_backward
 * (fps.cu:360-404), torch_point_ops_fps::gather_points_backward
 * (fps.cpp:161).
 *   grad_out (B,C,M), idx (B,M) int64, grad_points (B,C,N):
 *   zeros + scatter-add of grad_out at idx (duplicates sum).
 *   workspace: tpo_gather_bwd_workspace_size(B, N) bytes.
 */
int64_t tpo_gather_bwd_workspace_size(int64_t B, int64_t N);
int tpo_gather_bwd(int dtype, const void* grad_out, const int64_t* idx,
                   int64_t B, int64_t C, int64_t N, int64_t M,
                   void* grad_points, void* workspace, int64_t workspace_bytes,
                   void* stream);

/*
 * Earth mover's distance (approximate matching).
 *
 * tpo_emd_fwd replaces emd_cuda_forward (emd.cu:305-347: approxmatch
 * emd.cu:18-183 + matchcost emd.cu:187-230), the CUDA kernel of
 * torch_point_ops_emd::emd_forward (emd.cpp:32).
 *   xyz1 (B,n,3), xyz2 (B,m,3) -> cost (B) (the matching cost before the
 *   Python wrapper's division by n) and match (B,m,n).  F32/F64/F16.
 *   n == 0 or m == 0: cost = 0 and match is empty (emd.cu:313-318).
 *   Deterministic; within a tolerance of the reference (its exponential is
 *   CUDA's, this one is ROCm's, and the sums run in another order).
 * tpo_emd_bwd replaces emd_cuda_backward (emd.cu:349-389: matchcostgrad1
 * emd.cu:234-257 + matchcostgrad2 emd.cu:261-303), the kernel of
 * torch_point_ops_emd::emd_backward (emd.cpp:33).
 *   grad_cost (B), match (B,m,n) -> grad_xyz1 (B,n,3), grad_xyz2 (B,m,3).
 * Both take a workspace of tpo_emd_workspace_size(dtype, B, n, m) bytes,
 * 256-byte aligned (0 bytes when B, n or m is 0).  B < 2^31; n, m < 2^30.
 */
int64_t tpo_emd_workspace_size(int dtype, int64_t B, int64_t n, int64_t m);
int tpo_emd_fwd(int dtype, const void* xyz1, const void* xyz2, int64_t B,
                int64_t n, int64_t m, void* cost, void* match,
                void* workspace, int64_t workspace_bytes, void* stream);
int tpo_emd_bwd(int dtype, const void* grad_cost, const void* xyz1,
                const void* xyz2, const void* match, int64_t B, int64_t n,
                int64_t m, void* grad_xyz1, void* grad_xyz2,
                void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* TPO_H */
