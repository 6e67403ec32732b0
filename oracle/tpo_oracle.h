/*
 * tpo_oracle.h -- CPU oracle for the torch-point-ops nearest-neighbour path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the parity tests,
 * the smoke test and the bench's CPU-baseline leg compare against.  The
 * product (libtpo_hip.so + the torch_point_ops package) never links, loads
 * or calls it.
 *
 * Two families of functions live here:
 *   tpo_ref_*  restate the reference's CUDA-dispatch semantics (the behaviour
 *              the HIP kernels must reproduce): argmin/top-K tie rules, the
 *              fp16 per-operation rounding of c10::Half, the FMA order the
 *              reference's compiler contracts its distance sums into, the FPS
 *              skip rule and its tree-reduction tie order.
 *   tpo_cpu_*  restate the reference's own C++ CPU kernels (knn.cpp, fps.cpp)
 *              and are used only as the timed CPU baseline.
 *
 * dtype codes: 0 = float32, 1 = float64, 2 = float16 (IEEE binary16 bits in
 * uint16_t), 3 = bfloat16 (bits in uint16_t).  Index outputs follow the
 * reference: chamfer idx int32, knn idx int64, fps idx int64.
 *
 * Return value: 0 on success, negative on bad arguments.
 */
#ifndef TPO_ORACLE_H
#define TPO_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { TPO_REF_F32 = 0, TPO_REF_F64 = 1, TPO_REF_F16 = 2, TPO_REF_BF16 = 3 };

/* binary16 <-> binary32 conversions (round-to-nearest-even, subnormals kept) */
uint16_t tpo_ref_f32_to_f16(float f);
float tpo_ref_f16_to_f32(uint16_t h);
uint16_t tpo_ref_f32_to_bf16(float f);
float tpo_ref_bf16_to_f32(uint16_t h);
void tpo_ref_f32_to_f16_array(const float* in, uint16_t* out, int64_t n);
void tpo_ref_f16_to_f32_array(const uint16_t* in, float* out, int64_t n);
/* Number of float bit patterns for which the oracle's direct binary16
   rounding (used by every float16 operation) differs from
   tpo_ref_f16_to_f32(tpo_ref_f32_to_f16(x)); 0 when they agree everywhere. */
int64_t tpo_ref_f16_round_check(void);

/* Chamfer: chamfer.cu:36-167 (forward), chamfer.cu:200-234 (backward). */
int tpo_ref_chamfer_fwd(int dtype, const void* xyz1, const void* xyz2,
                        int64_t B, int64_t N, int64_t M,
                        void* dist1, void* dist2, int32_t* idx1, int32_t* idx2);
/* accum_f64 != 0: sum every per-pair contribution (computed in the dtype as
   the reference does) in double, then round once -- the exact value the
   atomics approximate in some order.  accum_f64 == 0: accumulate in the dtype
   in the sequential order direction 1 then direction 2. */
int tpo_ref_chamfer_bwd(int dtype, const void* xyz1, const void* xyz2,
                        const int32_t* idx1, const int32_t* idx2,
                        const void* gd1, const void* gd2,
                        int64_t B, int64_t N, int64_t M,
                        void* gxyz1, void* gxyz2, int accum_f64);

/* KNN: knn.cu:16-227 kernels V0-V3, mink.cuh:77-265, dispatch.cuh:106-147.
   version < 0 selects automatically; an invalid explicit version is replaced
   by the automatic choice (knn.cu:332-338).  Outputs are fully written:
   zeros where the reference leaves its zero-initialised outputs untouched. */
int tpo_ref_knn_choose_version(int64_t D, int64_t K, int version);
int tpo_ref_knn_fwd(int dtype, const void* p1, const void* p2,
                    const int64_t* len1, const int64_t* len2,
                    int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K,
                    int norm, int version, int64_t* idxs, void* dists);
/* knn.cu:400-466. accum_f64 as for chamfer. */
int tpo_ref_knn_bwd(int dtype, const void* p1, const void* p2,
                    const int64_t* len1, const int64_t* len2,
                    const int64_t* idxs, int norm, const void* grad_dists,
                    int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K,
                    void* gp1, void* gp2, int accum_f64);

/* FPS: fps.cu:56-60 (block size), fps.cu:100-214 (kernel), fps.cu:273-315. */
int tpo_ref_fps_block_size(int64_t n);
int tpo_ref_fps(int dtype, const void* pts, int64_t B, int64_t N, int64_t m,
                int64_t* idx);
/* Closed form of the reference's tie order: lower rank wins a tie of the
   running min-distance (bit-reversed thread id, then position in the
   thread's stride loop).  Used to cross-check the literal tree reduction. */
int64_t tpo_ref_fps_rank(int64_t k, int64_t n);

/* gather_points: fps.cu:63-98 */
int tpo_ref_gather_fwd(int dtype, const void* pts, const int64_t* idx,
                       int64_t B, int64_t C, int64_t N, int64_t M, void* out);
int tpo_ref_gather_bwd(int dtype, const void* grad_out, const int64_t* idx,
                       int64_t B, int64_t C, int64_t N, int64_t M,
                       void* grad_pts, int accum_f64);

/* Earth mover's distance (approximate matching): emd.cu:18-303.
   Forward writes cost[B] (the raw matchcost, before the module's division
   by n) and match[B][m][n]; backward writes grad_xyz1[B][n][3] and
   grad_xyz2[B][m][3] from grad_cost[B] and match.  float16 runs in float with
   half storage of the remain/ratio/match arrays, as the reference does.  The
   exponentials come from the C library (exp/expf): parity with the reference
   is within a tolerance, not bit-exact. */
int tpo_ref_emd_fwd(int dtype, const void* xyz1, const void* xyz2, int64_t B,
                    int64_t n, int64_t m, void* cost, void* match);
int tpo_ref_emd_bwd(int dtype, const void* grad_cost, const void* xyz1,
                    const void* xyz2, const void* match, int64_t B, int64_t n,
                    int64_t m, void* grad1, void* grad2);

/* Reference CPU kernels: knn.cpp:30-164, fps.cpp:18-141 (the CPU dispatch
   key's semantics: no FMA contraction, knn idx padding -1, FPS with
   FLT_MAX-style initial distances and selected-point exclusion).  They check
   the product's CPU kernels and are the timed CPU baseline.  dtype 0/1/2.
   nthreads > 1 splits independent rows (knn forward) or clouds (knn
   backward, fps) over OpenMP threads; results do not depend on it. */
int tpo_cpu_knn_fwd(int dtype, const void* p1, const void* p2,
                    const int64_t* len1, const int64_t* len2,
                    int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K,
                    int norm, int64_t* idxs, void* dists, int nthreads);
int tpo_cpu_knn_bwd(int dtype, const void* p1, const void* p2,
                    const int64_t* len1, const int64_t* len2,
                    const int64_t* idxs, int norm, const void* grad_dists,
                    int64_t N, int64_t P1, int64_t P2, int64_t D, int64_t K,
                    void* gp1, void* gp2, int nthreads);
int tpo_cpu_fps(int dtype, const void* pts, int64_t B, int64_t N, int64_t m,
                int64_t* idx, int nthreads);
int tpo_cpu_gather_fwd(int dtype, const void* pts, const int64_t* idx, int64_t B,
                       int64_t C, int64_t N, int64_t M, void* out);
int tpo_cpu_gather_bwd(int dtype, const void* grad_out, const int64_t* idx,
                       int64_t B, int64_t C, int64_t N, int64_t M,
                       void* grad_pts);

#ifdef __cplusplus
}
#endif
#endif
