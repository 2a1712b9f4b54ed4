/*
 * skmetal_hip.h -- C ABI of libskmetal_hip.so, the MI355X (gfx950) drop-in
 * for libSkMetalBridge.dylib on skmetal's KMeans fit/predict path.
 *
 * Conventions (unchanged from the reference's ctypes binding,
 * skmetal/_bridge.py:78-142, 345-363, 576-639):
 *   - size_t arguments are 64-bit (Swift Int in the reference);
 *   - X and centroids are float32, C-contiguous, row-major [n x d] / [k x d];
 *   - labels ("assignments") are 32-bit integers in [0, k);
 *   - the caller owns every buffer; no pointer is retained after a call
 *     returns, and every call is synchronous (results are in the caller's
 *     arrays on return);
 *   - 0 means success; a non-zero return is one of the SKMETAL_E* codes below
 *     (the reference returned 1 for every failure) and the message is
 *     available from skmetal_hip_last_error().  The library never aborts.
 *   - calls are serialised by an internal lock, so concurrent callers
 *     (ctypes releases the GIL) are safe.
 */
#ifndef SKMETAL_HIP_H
#define SKMETAL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__) || defined(__clang__)
#define SKMETAL_API __attribute__((visibility("default")))
#else
#define SKMETAL_API
#endif

#define SKMETAL_OK 0
#define SKMETAL_EINVAL 1   /* bad argument (null pointer, zero size, k > n ...) */
#define SKMETAL_ENODEV 2   /* no usable gfx950 device / HIP runtime failed to start */
#define SKMETAL_ENOMEM 3   /* device or pinned host allocation failed */
#define SKMETAL_ELAUNCH 4  /* kernel launch failed */
#define SKMETAL_EHIP 5     /* any other HIP runtime error */
#define SKMETAL_ERANGE 6   /* a size exceeds what the library supports */
#define SKMETAL_ENOSYS 7   /* a registry name outside the KMeans path (not provided) */

/* ---- set-up: skmetal_bridge/Sources/SkMetalBridgeC/include/bridge.h:11-12,60;
 *      Bridge.swift:19-48,52-144; bound at skmetal/_bridge.py:352-363 ---- */

/* Create the device context (device 0 of the visible devices).  Idempotent. */
SKMETAL_API int skmetal_init(void);

/* Load and run every kernel of the path once on a tiny problem. */
SKMETAL_API int skmetal_warmup(void);

/* Device name, max threads per block, unified-memory flag (0 on MI355X),
 * and total HBM bytes.  Replaces Bridge.swift:25-48 (bridge.h:12). */
SKMETAL_API int skmetal_device_info(char* name, int name_capacity, size_t* max_threads,
                        uint8_t* has_unified_memory, uint64_t* recommended_working_set_size);

/* ---- the KMeans path ---- */

/* E-step only: assignments[i] = argmin_j ||c_j||^2 - 2 x_i.c_j, lowest index on
 * ties, evaluated on X as given.  Replaces skmetal_kmeans_assign
 * (bridge.h:37; KMeansBridge.swift:138-181; _bridge.py:111-119, 576-578). */
SKMETAL_API int skmetal_kmeans_assign(const void* X, const void* centroids, void* assignments,
                          size_t n, size_t d, size_t k);

/* Lloyd loop with the reference's contract (KMeansBridge.swift:187-320): up
 * to max_iter steps; after each, the loop stops when the fp32 root of the
 * largest squared centre shift, max_j ||c_j_new - c_j_old||^2, is below tol
 * (:306-310; tol as the caller's estimator passes it, tol <= 0 never stops
 * early).  There is no label-based stop and no final E-step: assignments
 * (out, 32-bit) are the labels of the last step's E-step and centroids (in:
 * initial centres, out: the last step's centres, caller coordinates) those it
 * produced; *n_iter_out = steps run.  With max_iter = 0 nothing is written
 * but *n_iter_out = 0.  Each step is this library's: distances on X centred
 * on its column mean, empty clusters relocated as sklearn does (the reference
 * set them to 0).  num_groups is accepted for ABI compatibility and ignored
 * (the reference sized Metal threadgroup partials with it).  Replaces
 * skmetal_kmeans_batch_fused (bridge.h:39; _bridge.py:120-132, 591-617).
 * scikit-learn's stopping rules are those of skmetal_hip_kmeans_fit below. */
SKMETAL_API int skmetal_kmeans_batch_fused(const void* X, void* centroids, void* assignments,
                               size_t n, size_t d, size_t k, size_t num_groups,
                               size_t max_iter, float tol, int32_t* n_iter_out);

/* sum_i ||x_i - c_{label_i}||^2 (fp64 accumulation, returned as float), or
 * -1.0f on failure.  Replaces skmetal_kmeans_inertia (KMeansBridge.swift:324-373,
 * bound lazily at _bridge.py:627-639; absent from the reference's bridge.h). */
SKMETAL_API float skmetal_kmeans_inertia(const void* X, const void* centroids, const void* assignments,
                             size_t n, size_t d, size_t k);

/* dists[i] = ||x_i - c_{label_i}||^2 (fp32).  Replaces skmetal_compute_mindists
 * (bridge.h:45; KMeansBridge.swift:89-134; _bridge.py:133-142, 620-624). */
SKMETAL_API int skmetal_compute_mindists(const void* X, const void* centroids, const void* assignments,
                             void* dists, size_t n, size_t d, size_t k);

/* C = alpha op(A) op(B) + beta C in fp32, row-major A [M x K] (or [K x M] when
 * transpose_A), B [K x N] (or [N x K]), C [M x N]; with beta == 0 C is
 * write-only.  rocBLAS sgemm on the library's stream (librocblas is opened on
 * the first call).  Replaces skmetal_gemm (bridge.h:14-19; the MPS matrix
 * multiply bound at skmetal/_bridge.py:143-155 and called by
 * skmetal/_bridge.py:499-560), which skmetal's MetalKMeans.transform uses for
 * x.c^T (skmetal/estimators/cluster.py:135-146). */
SKMETAL_API int skmetal_gemm(const void* A, const void* B, void* C, size_t M, size_t N, size_t K, float alpha,
                             float beta, int transpose_A, int transpose_B);

/* ---- the rest of skmetal's ctypes registry (skmetal/_bridge.py:107-345) ----
 * skmetal's loader binds every registry name when the library loads
 * (skmetal/_bridge.py:345-349), so the names outside the KMeans path are
 * exported; each returns SKMETAL_ENOSYS with a message naming it, and
 * skmetal's wrappers raise RuntimeError("<name> failed with code 7").  The
 * argument lists follow the registry's argtypes. */
SKMETAL_API int skmetal_pairwise_distance(const void* X, void* D, size_t n, size_t d);
SKMETAL_API int skmetal_scaler_fit(const void* X, void* mean_out, void* var_out, size_t n, size_t d);
SKMETAL_API int skmetal_column_minmax(const void* X, void* min_out, void* max_out, size_t n, size_t d);
SKMETAL_API int skmetal_fista_fit(const void* X, const void* y, void* w, size_t n, size_t d, float alpha,
                                  float l1_ratio, float tol, int32_t max_iter, int32_t* n_iter_out);
SKMETAL_API int skmetal_column_transform(const void* input, void* output, const void* center, const void* scale,
                                         size_t n, size_t d);
SKMETAL_API int skmetal_sv_init(void* parent, size_t n);
SKMETAL_API int skmetal_sv_hook(void* parent, const void* edges, size_t n, size_t m);
SKMETAL_API int skmetal_sv_shortcut(void* parent, size_t n);
SKMETAL_API int skmetal_knn_vote_classify(const void* indices, const void* train_labels, void* predictions,
                                          size_t n, size_t k, size_t n_classes);
SKMETAL_API int skmetal_knn_vote_regress(const void* indices, const void* train_targets, void* predictions,
                                         size_t n, size_t k, size_t n_outputs);
SKMETAL_API int skmetal_knn_vote_classify_weighted(const void* indices, const void* weights, const void* train_labels,
                                                   void* predictions, size_t n, size_t k, size_t n_classes);
SKMETAL_API int skmetal_knn_vote_regress_weighted(const void* indices, const void* weights, const void* train_targets,
                                                  void* predictions, size_t n, size_t k, size_t n_outputs);
SKMETAL_API int skmetal_knn_tiled_kneighbors(const void* Q, const void* X, void* out_indices, void* out_dists,
                                             size_t nq, size_t nx, size_t d, size_t k, size_t tile, int32_t metric);
SKMETAL_API int skmetal_rbf_kernel_square(const void* X, void* K, float gamma, size_t n, size_t d);
SKMETAL_API int skmetal_rbf_kernel_cross(const void* X, const void* Y, void* K, float gamma, size_t n, size_t m,
                                         size_t d);
SKMETAL_API int skmetal_tree_predict_all(const void* X, const void* feature, const void* threshold,
                                         const void* left, const void* right, const void* value,
                                         const void* tree_offsets, const void* value_offsets, const void* n_nodes,
                                         const void* weights, void* out, size_t n, size_t d, size_t n_trees);
SKMETAL_API int skmetal_svc_predict_binary(const void* X, const void* sv, const void* dual_coef,
                                           const void* intercept, void* out, size_t n, size_t n_sv, size_t d,
                                           float gamma);
SKMETAL_API int skmetal_logreg_irls_fit(const void* X, const void* y, void* w, float C, float tol, int32_t max_iter,
                                        int32_t fit_intercept, size_t n, size_t d, int32_t* n_iter_out);
SKMETAL_API int skmetal_logreg_lbfgs_fit(const void* X, const void* y, void* w, float C, float tol, int32_t max_iter,
                                         int32_t fit_intercept, size_t n, size_t d, int32_t* n_iter_out);
SKMETAL_API int skmetal_ridge_fit_solve(const void* X, const void* y, void* coef, void* intercept, float alpha,
                                        size_t n, size_t d);
SKMETAL_API int skmetal_multinomial_lbfgs_fit(const void* X, const void* y, void* W, float C, float tol,
                                              int32_t max_iter, size_t n, size_t d, size_t n_classes,
                                              int32_t* n_iter_out);
SKMETAL_API int skmetal_minmax_transform(const void* X, void* X_out, const void* min_vals, const void* max_vals,
                                         size_t n, size_t d, float feature_min, float feature_max);
SKMETAL_API int skmetal_convert_f32_to_f16(const void* input, void* output, size_t n);
SKMETAL_API int skmetal_convert_f16_to_f32(const void* input, void* output, size_t n);
SKMETAL_API int skmetal_gemm_f16(const void* A, const void* B, void* C, size_t M, size_t N, size_t K);

/* ---- additions without a counterpart in the reference ---- */

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (tight serving loops, harnesses that forbid hipMalloc) and already
 * hold X, the centres and the labels in device memory:
 * skmetal_kmeans_batch_fused's loop contract on those caller-owned DEVICE
 * buffers, with no hipMalloc, hipFree or allocating library call.  It is not
 * for use under HIP graph capture: it runs on the library's own stream,
 * clears its loop state and labels with hipMemsetAsync and waits for the
 * device before it returns.  X is [n x d]
 * fp32 in device memory, used as given (not centred); centroids is [k x d] in
 * device memory, in/out; assignments is [n] int32 in device memory, out;
 * *n_iter_out (host) = steps run.  Every other buffer comes from a static
 * 32 MiB device array per GPU, whose address skmetal_init takes: skmetal_init
 * must have succeeded first.  Limits: k <= 64, d one of 4, 8, 16, 32, 48, 64,
 * 80, 100 (the fused kernels' row lengths), n <= 4,194,304; beyond them the
 * call returns SKMETAL_ERANGE.  Calls are serialised by the library's lock;
 * calls that overlap on one GPU from different processes each have their own
 * array.  The call is synchronous (it waits for the device before it
 * returns). */
SKMETAL_API int skmetal_hip_kmeans_batch_fused_noalloc(const float* X, float* centroids, int32_t* assignments,
                                                      size_t n, size_t d, size_t k, size_t max_iter, float tol,
                                                      int32_t* n_iter_out);

/* Message of the last failure on the calling thread ("" if none). */
SKMETAL_API const char* skmetal_hip_last_error(void);

/* Release the device buffers the library keeps cached between calls. */
SKMETAL_API int skmetal_hip_release_cache(void);

/* Whole Lloyd fit with sklearn KMeans(init=centroids, n_init=1,
 * algorithm="lloyd") semantics, plus the final inertia (fp64), with a single
 * upload of X: X centred on its column mean for the distance evaluations; the
 * loop stops when sum_j ||c_j_new - c_j_old||^2 <= tol (sklearn's absolute
 * `_tol`: mean feature variance x estimator tol), with SKMETAL_FIT_STRICT also
 * on strict label convergence (pass it for sklearn semantics), or after
 * max_iter steps; empty clusters are relocated as sklearn does; a final E-step
 * makes the labels those of the returned centres; *n_iter_out = sklearn's
 * n_iter_. */
#define SKMETAL_FIT_STRICT 1
SKMETAL_API int skmetal_hip_kmeans_fit(const float* X, float* centroids, int32_t* labels,
                           size_t n, size_t d, size_t k, size_t max_iter, double tol,
                           int flags, int32_t* n_iter_out, double* inertia_out);

/* Device-resident Lloyd handle: X is uploaded (and optionally centred) once
 * and stays in HBM across calls; used for timing a fixed number of
 * iterations and for step-by-step checks.  Not thread-safe per handle. */
typedef struct skmetal_hip_lloyd skmetal_hip_lloyd;

SKMETAL_API int skmetal_hip_lloyd_create(size_t n, size_t d, size_t k, skmetal_hip_lloyd** out);
SKMETAL_API int skmetal_hip_lloyd_destroy(skmetal_hip_lloyd* h);
/* Upload X [n x d]; center != 0 subtracts the column mean on the device. */
SKMETAL_API int skmetal_hip_lloyd_load(skmetal_hip_lloyd* h, const float* X, int center);
/* Set the centres [k x d] (caller coordinates). */
SKMETAL_API int skmetal_hip_lloyd_set_centers(skmetal_hip_lloyd* h, const float* C);
/* Run exactly `iters` Lloyd steps (E-step + M-step, no convergence stop;
 * empty clusters are still relocated).  If ms_out is not NULL it receives
 * the elapsed time of the steps measured with HIP events on the handle's
 * stream.  If kernel_ms is not NULL (iters <= 4096) each step is also
 * bracketed by HIP events and kernel_ms[0..2] receive the average time per
 * step (ms) of the E-step kernel (the fused E-step + sums kernel when the
 * handle uses it), of the separate update kernels (0 when fused) and of the
 * finalize. */
SKMETAL_API int skmetal_hip_lloyd_iterate(skmetal_hip_lloyd* h, size_t iters, float* ms_out,
                                          float* kernel_ms);
/* sklearn loop (see skmetal_hip_kmeans_fit) from the current centres,
 * including the final E-step and inertia. */
SKMETAL_API int skmetal_hip_lloyd_run(skmetal_hip_lloyd* h, size_t max_iter, double tol, int flags,
                          int32_t* n_iter_out, double* inertia_out);
/* Greedy k-means++ seeding of the handle's centres from the loaded X
 * (centred if it was loaded with center != 0, as scikit-learn's fit seeds on
 * centred X): scikit-learn's _kmeans_plusplus with unit sample weights
 * (sklearn/cluster/_kmeans.py:174-260), the random numbers drawn by the
 * caller in scikit-learn's order: first_index = the first centre's row
 * (RandomState.choice(n, p=w / w.sum()), :225), uniforms = the
 * (k - 1) x n_local_trials values of the k - 1 calls
 * RandomState.uniform(size=n_local_trials) (:243), row-major.  The k chosen
 * rows become the current centres and their indices go to indices_out [k].
 * n_local_trials in [1, 64]; scikit-learn's default is 2 + int(ln k).
 * No counterpart in the reference (skmetal seeded with k-means|| on the host,
 * skmetal/estimators/cluster.py:70-116); this replaces the scikit-learn
 * seeding the estimator would otherwise run on the CPU. */
SKMETAL_API int skmetal_hip_lloyd_plusplus(skmetal_hip_lloyd* h, size_t n_local_trials, int64_t first_index,
                                           const double* uniforms, int64_t* indices_out);
/* The same seeding on X [n x d] as given (no centring), like
 * sklearn.cluster.kmeans_plusplus: indices_out [k] receives the chosen rows. */
SKMETAL_API int skmetal_hip_kmeans_plusplus(const float* X, size_t n, size_t d, size_t k, size_t n_local_trials,
                                            int64_t first_index, const double* uniforms, int64_t* indices_out);
/* KMeans.transform: out[i * k + j] = ||x_i - c_j|| (float32, [n x k]) as
 * scikit-learn computes it for float32 data (euclidean_distances,
 * sklearn/cluster/_kmeans.py:1124-1148; sklearn/metrics/pairwise.py:582-652):
 * the fp64 expanded distance cast to fp32, negatives set to 0, fp32 square
 * root.  Replaces the reference's transform through skmetal_gemm
 * (skmetal/estimators/cluster.py:135-146; _bridge.py:499-563), which formed
 * the same expression in fp32. */
SKMETAL_API int skmetal_hip_kmeans_transform(const float* X, const float* centroids, float* out, size_t n, size_t d,
                                             size_t k);
/* out[d] = numpy's float32 np.var(X, axis=0) of a C-ordered X [n x d], bit for
 * bit: the column variances scikit-learn's _tolerance averages
 * (sklearn/cluster/_kmeans.py:279-287).  Host threads run numpy's row-order
 * fp32 chains over column ranges, two passes over X without temporaries
 * (numpy's own np.var makes four, and a copy of X).  Needs no device.  No
 * counterpart in the reference. */
SKMETAL_API int skmetal_hip_column_variance(const float* X, size_t n, size_t d, float* out);
/* Largest |x| of the loaded X (after the centring, if any), NaN counted as
 * +inf: a finite value means X holds no NaN or infinity, so a caller can skip
 * its own pass over X.  A non-finite value can also come from a centring
 * that overflowed, so the caller then checks X itself. */
SKMETAL_API int skmetal_hip_lloyd_max_abs(skmetal_hip_lloyd* h, float* out);
/* One k-means|| round on the loaded X: the squared distance of every row to
 * its nearest candidate so far, kept on the device and lowered with the m new
 * candidate rows (indices into X); reset = 1 starts from +inf (required on the
 * first call).  dists_out [n] (nullable) receives the result.  Replaces the
 * per-round skmetal_kmeans_assign + skmetal_compute_mindists pair of
 * MetalKMeans._kmeans_parallel_init (skmetal/estimators/cluster.py:92-93),
 * each of which uploads X again; the distance to the assigned candidate is the
 * minimum over the candidates.  Distances are scikit-learn's fp32 form (fp64
 * expanded distance, cast to fp32, negatives to 0), as in the k-means++ entry
 * points. */
SKMETAL_API int skmetal_hip_lloyd_mindists(skmetal_hip_lloyd* h, const int64_t* rows, size_t m, int reset,
                                           float* dists_out);
/* numpy's legacy RandomState.choice(n, size, replace=False, p=w / w.sum())
 * over the loaded rows, on the device, for fp32 weights w: weights = 0 takes
 * the k-means|| distances of skmetal_hip_lloyd_mindists floored at 1e-30
 * (numpy maximum), as MetalKMeans._kmeans_parallel_init draws its candidates
 * (skmetal/estimators/cluster.py:94-98); weights = 1 takes unit weights, as
 * scikit-learn's init="random" (sklearn/cluster/_kmeans.py:1010-1013).
 * sample_prepare forms p in numpy's arithmetic (fp32 sum in numpy's pairwise
 * order, fp32 quotient, fp64) and returns the fp64 sum of p and the count of
 * p > 0, which choice checks before drawing.  Each sample_draw is one of
 * choice's passes: p is zeroed at the n_zero rows found so far, then
 * rows_out[t] = searchsorted(cumsum(p) / cumsum(p)[-1], uniforms[t],
 * side="right") with numpy's sequential fp64 cumsum, for the m uniforms the
 * caller drew with rand(size - found).  The row is found on a cumsum of
 * another order and kept when it is provably the same; the rest (about
 * 4 n 2^-53 of the draws) are searched on numpy's own cumsum, every draw with
 * exact = 1; exact = 2 gives the proof a margin of at least 1/(4n), so that
 * about half the draws take each search (for tests of both in one pass).
 * *n_exact_out (nullable) = the draws searched that way.  The caller drops
 * repeated rows and draws again, as choice does. */
SKMETAL_API int skmetal_hip_lloyd_sample_prepare(skmetal_hip_lloyd* h, int weights, double* p_sum_out,
                                                 int64_t* nonzero_out);
SKMETAL_API int skmetal_hip_lloyd_sample_draw(skmetal_hip_lloyd* h, const int64_t* zero_rows, size_t n_zero,
                                              const double* uniforms, size_t m, int64_t* rows_out, int exact,
                                              int* n_exact_out);
/* *fused & 3 = 0 when a step runs as separate E-step and update kernels, 1
 * when as one fused E-step + sums kernel with the E-step on fp32 MFMA
 * (k <= 64, d <= 100), 2 when that kernel's E-step and sums run on bf16 MFMAs
 * over an exact three-part bf16 split of x and c with fp32 accumulation
 * (d >= 17, finite data with max |x| 0 or in [2^-50, 2^60]); *fused & 4 = the
 * separate E-step kernel (generic path, final E-step, assign) uses the same
 * split; *partials = per-step partial sums the finalize reduces. */
SKMETAL_API int skmetal_hip_lloyd_info(skmetal_hip_lloyd* h, int* fused, int* partials);
SKMETAL_API int skmetal_hip_lloyd_get_centers(skmetal_hip_lloyd* h, float* C);
SKMETAL_API int skmetal_hip_lloyd_get_labels(skmetal_hip_lloyd* h, int32_t* labels);
/* Inertia of the current labels against the current centres (fp64). */
SKMETAL_API int skmetal_hip_lloyd_inertia(skmetal_hip_lloyd* h, double* out);

#ifdef __cplusplus
}
#endif

#endif /* SKMETAL_HIP_H */
